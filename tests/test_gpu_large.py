"""GPU parity beyond 32-bit element counts: every batched entry whose kernels index with 64-bit offsets runs
once over more than 2^32 elements (17-69 GB of HBM per case), and the Q8 embedding gather on both sides of
the point where its launcher leaves the flat-piece kernel (32-bit dword indices) for the row kernel.

The outputs are checked bit for bit on sampled rows, against the oracle or a closed form: the first rows, the
rows around the 2^31 and 2^32 element (or dword) boundaries and the last rows.  The element-wise entry is
checked in full against torch's IEEE addition on the device.  A case is skipped when the device has not
the memory it needs free.
"""
from __future__ import annotations

import numpy as np
import pytest

from tests import common as C

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

GB = 1 << 30


@pytest.fixture(scope="module")
def ops():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a visible MI355X")
    from v7multiplikator_amd import _lib
    from v7multiplikator_amd import ops as _ops
    _lib.load()
    return _ops


@pytest.fixture(autouse=True)
def release_memory():
    yield
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def need(nbytes):
    free, _ = torch.cuda.mem_get_info()
    if free < nbytes + 4 * GB:
        pytest.skip(f"needs {nbytes / GB:.0f} GiB of free device memory, {free / GB:.0f} GiB free")


def same(a, b):
    a, b = np.asarray(a), np.asarray(b)
    if a.dtype.kind == "f":
        return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))
    return a.shape == b.shape and np.array_equal(a, b)


def sample_rows(rows, row_len):
    """First and last rows, and the rows holding elements 2^31 and 2^32 (with a neighbour on each side)."""
    picks = {0, 1, rows - 2, rows - 1}
    for e in (1 << 31, 1 << 32):
        r = e // row_len
        picks.update(x for x in (r - 1, r, r + 1) if 0 <= x < rows)
    return np.array(sorted(picks), dtype=np.int64)


def host_rows(t, rows):
    torch.cuda.synchronize()
    return np.stack([t[int(r)].cpu().numpy() for r in rows])


def gen(seed):
    g = torch.Generator(device="cuda")
    g.manual_seed(seed)
    return g


def test_add_inplace_past_2_pow_32_elements(ops):
    """x += y over 2^32 + 7 floats: the float4 kernel's 64-bit block base and the 3-element tail."""
    n = (1 << 32) + 7
    need(3 * 4 * n)
    g = gen(901)
    x = torch.empty(n, dtype=torch.float32, device="cuda").normal_(generator=g)
    y = torch.empty(n, dtype=torch.float32, device="cuda").normal_(generator=g)
    want = x + y
    ops.add_inplace(x, y)
    torch.cuda.synchronize()
    assert torch.equal(x.view(torch.int32), want.view(torch.int32))
    tail = slice(n - 11, n)
    assert same(x[tail].cpu().numpy(), (want[tail].cpu().numpy()))


def test_swiglu_q8_past_2_pow_32_elements(ops, oracle):
    """SwiGLU -> Q8 (GS 32) over [349526, 12288]: 4,294,975,488 elements, the flat kernel's 64-bit chunk
    offsets; sampled rows against the oracle."""
    rows, hidden = 349526, 12288
    need(2 * 4 * rows * hidden + rows * hidden + rows * hidden // 32 * 4)
    g = gen(902)
    gate = torch.empty((rows, hidden), dtype=torch.float32, device="cuda").normal_(0.0, 1.5, generator=g)
    up = torch.empty((rows, hidden), dtype=torch.float32, device="cuda").normal_(0.0, 1.5, generator=g)
    q, s = ops.swiglu_q8(gate, up, gs=32)
    pick = sample_rows(rows, hidden)
    wq, ws = oracle.swiglu_q8(host_rows(gate, pick), host_rows(up, pick), 32)
    assert same(host_rows(q, pick), wq) and same(host_rows(s, pick), ws)


def test_rmsnorm_quantize_past_2_pow_32_elements(ops, oracle):
    """RMSNorm -> Q8 (GS 64) over [1048577, 4096] (one row past 2^32 elements), then the fused-add form over
    the same rows; sampled rows against the oracle."""
    rows, dim = (1 << 20) + 1, 4096
    need(2 * 4 * rows * dim + rows * dim + rows * dim // 64 * 4)
    g = gen(903)
    x = torch.empty((rows, dim), dtype=torch.float32, device="cuda").normal_(generator=g)
    w = torch.from_numpy(C.norm_weight(904, dim)).cuda()
    pick = sample_rows(rows, dim)
    x_rows = host_rows(x, pick)
    q, s = ops.rmsnorm_quantize(x, w, eps=1e-6, gs=64)
    wq, ws = oracle.rmsnorm_quantize(x_rows, w.cpu().numpy(), 1e-6, 64)
    assert same(host_rows(q, pick), wq) and same(host_rows(s, pick), ws)
    a = torch.empty((rows, dim), dtype=torch.float32, device="cuda").normal_(generator=g)
    a_rows = host_rows(a, pick)
    ops.add_rmsnorm_quantize(x, a, w, eps=1e-6, gs=64, out_q=q, out_s=s)
    summed = oracle.add_inplace(x_rows, a_rows)
    wq, ws = oracle.rmsnorm_quantize(summed, w.cpu().numpy(), 1e-6, 64)
    assert same(host_rows(x, pick), summed)
    assert same(host_rows(q, pick), wq) and same(host_rows(s, pick), ws)


def test_fused_add_rmsnorm_past_2_pow_32_elements(ops, oracle):
    """residual += add, out = RMSNorm(residual) * w over [1048577, 4096]; sampled rows against the oracle."""
    rows, dim = (1 << 20) + 1, 4096
    need(3 * 4 * rows * dim)
    g = gen(905)
    r = torch.empty((rows, dim), dtype=torch.float32, device="cuda").normal_(generator=g)
    a = torch.empty((rows, dim), dtype=torch.float32, device="cuda").normal_(generator=g)
    w = torch.from_numpy(C.norm_weight(906, dim)).cuda()
    pick = sample_rows(rows, dim)
    r_rows, a_rows = host_rows(r, pick), host_rows(a, pick)
    o = ops.fused_add_rmsnorm(r, a, w, eps=1e-6)
    want_o, want_r = oracle.fused_add_rmsnorm(r_rows, a_rows, w.cpu().numpy(), 1e-6)
    assert same(host_rows(r, pick), want_r) and same(host_rows(o, pick), want_o)


def test_qk_rmsnorm_rope_past_2_pow_32_elements(ops, oracle):
    """Q/K RMSNorm+RoPE in place inside fused QKV rows of 6144 floats over 700,000 tokens (4.3e9 floats;
    32 + 8 heads of 128, positions cycling through an 8192-row table); sampled tokens against the oracle."""
    n, nq, nkv, hd = 700000, 32, 8, 128
    width = (nq + 2 * nkv) * hd
    need(4 * n * width)
    g = gen(907)
    qkv = torch.empty((n, width), dtype=torch.float32, device="cuda").normal_(generator=g)
    qw, kw = C.norm_weight(908, hd), C.norm_weight(909, hd)
    ct, st = oracle.rope_tables(8192, hd, 1e6)
    pos = (np.arange(n, dtype=np.int64) % 8192).astype(np.int32)
    pick = sample_rows(n, width)
    before = host_rows(qkv, pick)
    q = qkv[:, :nq * hd].view(n, nq, hd)
    k = qkv[:, nq * hd:(nq + nkv) * hd].view(n, nkv, hd)
    ops.qk_rmsnorm_rope(q, k, torch.from_numpy(qw).cuda(), torch.from_numpy(kw).cuda(), torch.from_numpy(ct).cuda(),
                        torch.from_numpy(st).cuda(), positions=torch.from_numpy(pos).cuda(), eps=1e-6)
    after = host_rows(qkv, pick)
    p = pos[pick]
    want_q = oracle.rmsnorm_rope(before[:, :nq * hd].reshape(-1, nq, hd), qw, ct, st, p, 1e-6)
    want_k = oracle.rmsnorm_rope(before[:, nq * hd:(nq + nkv) * hd].reshape(-1, nkv, hd), kw, ct, st, p, 1e-6)
    assert same(after[:, :nq * hd].reshape(-1, nq, hd), want_q)
    assert same(after[:, nq * hd:(nq + nkv) * hd].reshape(-1, nkv, hd), want_k)
    assert same(after[:, (nq + nkv) * hd:], before[:, (nq + nkv) * hd:])


def test_embedding_gather_on_both_sides_of_the_32_bit_dword_limit(ops):
    """Rows of 4096 codes (1024 dwords): 4,194,295 rows (2^32 - 9216 dwords of codes, a 68.7 GB output) still
    take the flat-piece kernel, 4,194,296 rows (2^32 - 8192 dwords) the row kernel; ids include invalid ones
    (rows of zeros).  Sampled rows against the closed form code * scale."""
    dim, vocab = 4096, 4096
    big = 4194296
    need(4 * big * dim + 8 * big)
    tq, ts = C.q8_table(910, vocab, dim)
    ids = C.rng(911).integers(0, vocab, big).astype(np.int32)
    for r, bad in ((5, -1), (2097152, vocab), (big - 3, 1 << 30), (big - 2, -7)):
        ids[r] = bad
    out = torch.empty((big, dim), dtype=torch.float32, device="cuda")
    d_ids, d_tq, d_ts = torch.from_numpy(ids).cuda(), torch.from_numpy(tq).cuda(), torch.from_numpy(ts).cuda()
    table = tq.astype(np.float32) * np.repeat(ts.reshape(vocab, dim // 64), 64, axis=1)
    for n in (big - 1, big):
        out[n - 4:n].fill_(float("nan"))
        ops.embedding_gather_q8(d_ids[:n], d_tq, d_ts, out=out[:n])
        pick = np.array(sorted({0, 1, 5, 2097151, 2097152, 2097153, 1048576, n - 3, n - 2, n - 1}), np.int64)
        got = host_rows(out, pick)
        sel = ids[pick]
        valid = (sel >= 0) & (sel < vocab)
        want = np.zeros((len(pick), dim), np.float32)
        want[valid] = table[sel[valid]]
        assert same(got, want), n


def test_quantize_q8_generic_rows_past_2_pow_32_elements(ops, oracle):
    """Q8 quantize (GS 64) of rows of 4100 floats (the general kernel: one thread per group, a 4-element tail
    group per row) over 1,047,553 rows = 4,294,967,300 elements; sampled rows against the oracle."""
    rows, row_len = 1047553, 4100
    need(4 * rows * row_len + rows * row_len + rows * 65 * 4)
    g = gen(912)
    x = torch.empty((rows, row_len), dtype=torch.float32, device="cuda").normal_(generator=g)
    q, s = ops.quantize_q8(x, gs=64)
    pick = sample_rows(rows, row_len)
    wq, ws = oracle.quantize(host_rows(x, pick), 64)
    assert same(host_rows(q, pick), wq) and same(host_rows(s, pick), ws)


def test_rmsnorm_past_2_pow_32_elements(ops, oracle):
    """out = RMSNorm(x) * w over [1048577, 4096]; sampled rows against the oracle."""
    rows, dim = (1 << 20) + 1, 4096
    need(2 * 4 * rows * dim)
    g = gen(913)
    x = torch.empty((rows, dim), dtype=torch.float32, device="cuda").normal_(generator=g)
    w = torch.from_numpy(C.norm_weight(914, dim)).cuda()
    o = ops.rmsnorm(x, w, eps=1e-6)
    pick = sample_rows(rows, dim)
    assert same(host_rows(o, pick), oracle.rmsnorm(host_rows(x, pick), w.cpu().numpy(), 1e-6))


def test_kv_pack_past_2_pow_32_elements(ops, oracle):
    """binary16 packing of [2097153, 2048] f32 rows (4.3e9 floats): the whole rows with one launch, then their
    K and V halves as the two sides of the one-launch pack; sampled rows against the oracle."""
    rows, width = 2097153, 2048
    need(4 * rows * width + 2 * rows * width)
    g = gen(915)
    src = torch.empty((rows, width), dtype=torch.float32, device="cuda").normal_(generator=g)
    pick = sample_rows(rows, width)
    src_rows = host_rows(src, pick)
    out = ops.kv_pack_f16(src)
    assert same(host_rows(out, pick).view(np.uint16), oracle.kv_pack_f16(src_rows))
    del out
    half = width // 2
    hk, hv = ops.kv_pack_f16_kv(src[:, :half], src[:, half:])
    assert same(host_rows(hk, pick).view(np.uint16), oracle.kv_pack_f16(src_rows[:, :half]))
    assert same(host_rows(hv, pick).view(np.uint16), oracle.kv_pack_f16(src_rows[:, half:]))


def test_qkv_stage_with_caches_past_2_pow_32_elements(ops, oracle):
    """The Q/K/V stage with a QKV bias, RoPE only (no norm weights) and binary16 K/V cache rows, in place
    inside 700,000 fused QKV rows of 6144 floats (4.3e9 floats; 32 + 8 + 8 heads of 128); sampled tokens
    against the oracle."""
    n, nq, nkv, hd = 700000, 32, 8, 128
    width = (nq + 2 * nkv) * hd
    need(4 * n * width + 2 * 2 * n * nkv * hd)
    g = gen(916)
    qkv = torch.empty((n, width), dtype=torch.float32, device="cuda").normal_(generator=g)
    qb, kb, vb = (C.normal(917 + i, (h * hd,), 0.5) for i, h in enumerate((nq, nkv, nkv)))
    ct, st = oracle.rope_tables(8192, hd, 1e6)
    pos = (np.arange(n, dtype=np.int64) * 7 % 8192).astype(np.int32)
    pick = sample_rows(n, width)
    before = host_rows(qkv, pick)
    kc = torch.empty((n, nkv, hd), dtype=torch.float16, device="cuda")
    vc = torch.empty((n, nkv, hd), dtype=torch.float16, device="cuda")
    k0, v0 = nq * hd, (nq + nkv) * hd
    ops.qkv_rope_stage(qkv[:, :k0].view(n, nq, hd), qkv[:, k0:v0].view(n, nkv, hd), qkv[:, v0:].view(n, nkv, hd),
                       torch.from_numpy(ct).cuda(), torch.from_numpy(st).cuda(), positions=torch.from_numpy(pos).cuda(),
                       q_bias=torch.from_numpy(qb).cuda(), k_bias=torch.from_numpy(kb).cuda(),
                       v_bias=torch.from_numpy(vb).cuda(), k_cache=kc, v_cache=vc)
    after = host_rows(qkv, pick)
    wq, wk, wv, wkc, wvc = oracle.qkv_stage(before[:, :k0].reshape(-1, nq, hd), before[:, k0:v0].reshape(-1, nkv, hd),
                                            before[:, v0:].reshape(-1, nkv, hd), None, None, qb, kb, vb, ct, st,
                                            pos[pick], 1e-6)
    assert same(after[:, :k0].reshape(-1, nq, hd), wq)
    assert same(after[:, k0:v0].reshape(-1, nkv, hd), wk)
    assert same(after[:, v0:].reshape(-1, nkv, hd), wv)
    assert same(host_rows(kc, pick).view(np.uint16), wkc)
    assert same(host_rows(vc, pick).view(np.uint16), wvc)


@pytest.mark.parametrize("stride", [(1 << 32) - 4, (1 << 32) + 4096])
def test_kv_pack_kv_with_row_strides_around_2_pow_32(ops, oracle, stride):
    """The one-launch K/V pack with a source row stride of 2^32 - 4 floats (the largest the 32-bit-stride kernel
    form takes) and of 2^32 + 4096 (the 64-bit form): two rows 17.2 GB apart."""
    need(4 * (stride + 2048))
    g = gen(920)
    flat = torch.empty(stride + 2048, dtype=torch.float32, device="cuda")
    flat[:2048].normal_(generator=g)
    flat[stride:].normal_(generator=g)
    k_src = flat.as_strided((2, 1024), (stride, 1))
    v_src = flat.as_strided((2, 1024), (stride, 1), 1024)
    hk, hv = ops.kv_pack_f16_kv(k_src, v_src)
    rows = np.stack([flat[:2048].cpu().numpy(), flat[stride:].cpu().numpy()])
    assert same(hk.cpu().numpy().view(np.uint16), oracle.kv_pack_f16(rows[:, :1024]))
    assert same(hv.cpu().numpy().view(np.uint16), oracle.kv_pack_f16(rows[:, 1024:]))
