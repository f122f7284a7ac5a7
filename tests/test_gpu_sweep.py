"""GPU parity over seeded random shapes: every batched entry against the oracle, bit for bit.

The fixed-shape tests pin the benchmark configurations and the reference validators' shapes; this
sweep draws the shape parameters at random inside each entry's contract (rows, row lengths that are
not multiples of the vector width, ragged quantization tails, every head_dim class, tables wider than
head_dim / 2, positions anywhere in the table) so that an indexing mistake that only shows at an
unusual shape fails here.  Each case names its parameters in the failure message.  V7G_SWEEP_CASES
(default 12) and V7G_SWEEP_SEED (default 0) widen or move the sweep, e.g. for a longer run by hand.
"""
from __future__ import annotations

import os

import numpy as np
import pytest

from tests import common as C

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

CASES = int(os.environ.get("V7G_SWEEP_CASES", "12"))
SEED = int(os.environ.get("V7G_SWEEP_SEED", "0"))


@pytest.fixture(scope="module")
def ops():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a visible MI355X")
    from v7multiplikator_amd import _lib
    from v7multiplikator_amd import ops as _ops
    _lib.load()
    return _ops


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def same(a, b):
    a, b = np.asarray(a), np.asarray(b)
    if a.shape != b.shape:
        return False
    if a.dtype.kind == "f":
        return np.array_equal(a.view(np.uint32), b.view(np.uint32))
    return np.array_equal(a, b)


def shapes(tag, draw):
    """CASES parameter sets from a generator seeded by the test's tag."""
    r = np.random.default_rng(sum(map(ord, tag)) * 7919 + SEED)
    return [draw(r) for _ in range(CASES)]


def test_sweep_fused_add_rmsnorm(ops, oracle):
    for rows, dim, eps in shapes("arn", lambda r: (int(r.integers(1, 48)), 8 * int(r.integers(1, 2049)),
                                                   float(r.choice([1e-6, 1e-5])))):
        res = C.normal(rows * 7 + dim, (rows, dim))
        add = C.normal(rows * 7 + dim + 1, (rows, dim))
        w = C.norm_weight(dim, dim)
        want_o, want_r = oracle.fused_add_rmsnorm(res, add, w, eps)
        rt = dev(res)
        got_o = host(ops.fused_add_rmsnorm(rt, dev(add), dev(w), eps=eps))
        assert same(got_o, want_o) and same(host(rt), want_r), (rows, dim, eps)


def test_sweep_one_wave_rows(ops, oracle):
    """More than 2048 rows of 264 to 1016 floats (one wave per row), a quarter of the cases: add+RMSNorm at every
    width % 8, RMSNorm and RMSNorm -> Q8 at width % 64."""
    def draw(r):
        return int(r.integers(2049, 3001)), 8 * int(r.integers(33, 128)), int(r.choice([32, 64]))

    for rows, dim, gs in shapes("wave_rows", draw)[:max(1, CASES // 4)]:
        res = C.normal(rows + dim, (rows, dim))
        add = C.normal(rows + dim + 1, (rows, dim))
        w = C.norm_weight(dim + 9, dim)
        want_o, want_r = oracle.fused_add_rmsnorm(res, add, w, 1e-6)
        rt = dev(res)
        got_o = host(ops.fused_add_rmsnorm(rt, dev(add), dev(w), eps=1e-6))
        assert same(got_o, want_o) and same(host(rt), want_r), (rows, dim)
        if dim % 64 == 0:
            assert same(host(ops.rmsnorm(dev(res), dev(w), eps=1e-6)), oracle.rmsnorm(res, w, 1e-6)), (rows, dim)
            wq, ws = oracle.rmsnorm_quantize(res, w, 1e-6, gs)
            gq, gsc = ops.rmsnorm_quantize(dev(res), dev(w), eps=1e-6, gs=gs)
            assert same(host(gq), wq) and same(host(gsc), ws), (rows, dim, gs)


def test_sweep_rmsnorm_and_quantize(ops, oracle):
    for rows, dim, gs, eps in shapes("rmsq", lambda r: (int(r.integers(1, 40)), 64 * int(r.integers(1, 257)),
                                                        int(r.choice([32, 64])), float(r.choice([1e-6, 1e-5])))):
        x = C.normal(rows * 13 + dim, (rows, dim), 2.0)
        w = C.norm_weight(dim + 3, dim)
        assert same(host(ops.rmsnorm(dev(x), dev(w), eps=eps)), oracle.rmsnorm(x, w, eps)), (rows, dim, eps)
        wq, ws = oracle.rmsnorm_quantize(x, w, eps, gs)
        gq, gsc = ops.rmsnorm_quantize(dev(x), dev(w), eps=eps, gs=gs)
        assert same(host(gq), wq) and same(host(gsc), ws), (rows, dim, gs, eps)
        add = C.normal(rows * 13 + dim + 1, (rows, dim))
        rt = dev(x)
        gq, gsc = ops.add_rmsnorm_quantize(rt, dev(add), dev(w), eps=eps, gs=gs)
        summed = oracle.add_inplace(x, add)
        wq, ws = oracle.rmsnorm_quantize(summed, w, eps, gs)
        assert same(host(rt), summed) and same(host(gq), wq) and same(host(gsc), ws), ("add", rows, dim, gs, eps)


def test_sweep_rmsnorm_rope(ops, oracle):
    def draw(r):
        hd = 32 * int(r.integers(2, 17))
        wide = bool(r.integers(0, 2))
        return int(r.integers(1, 24)), int(r.integers(1, 41)), hd, wide, int(r.integers(1, 300))

    for T, H, hd, wide, n_pos in shapes("rope", draw):
        table_hd = 2 * hd if wide else hd  # a wider table row than head_dim / 2 is allowed
        ct, st = oracle.rope_tables(n_pos, table_hd, 1e6 if hd % 64 == 0 else 1e4)
        pos = C.rng(T * H + hd).integers(0, n_pos, T).astype(np.int32)
        buf = C.normal(T + H + hd, (T, H, hd))
        w = C.norm_weight(hd + 5, hd)
        bt = dev(buf)
        ops.rmsnorm_rope_heads(bt, dev(w), dev(ct), dev(st), positions=dev(pos), eps=1e-6)
        assert same(host(bt), oracle.rmsnorm_rope(buf, w, ct, st, pos, 1e-6)), (T, H, hd, wide, n_pos)
        bt = dev(buf)
        ops.rope_only_heads(bt, dev(ct), dev(st), positions=dev(pos))
        assert same(host(bt), oracle.rope_only(buf, ct, st, pos)), ("rope only", T, H, hd, wide, n_pos)


def test_sweep_qk_in_fused_row(ops, oracle):
    """Q and K heads at random offsets inside one token row with a random (wider) token stride."""
    def draw(r):
        return (int(r.integers(1, 20)), int(r.integers(1, 17)), int(r.integers(1, 9)), 32 * int(r.integers(2, 9)),
                4 * int(r.integers(0, 9)))

    for T, nq, nkv, hd, pad in shapes("qk", draw):
        row = (nq + 2 * nkv) * hd + pad
        qkv = C.normal(T * row, (T, row))
        ct, st = oracle.rope_tables(T + 3, hd, 1e6)
        pos = np.arange(3, T + 3, dtype=np.int32)
        qw, kw = C.norm_weight(hd, hd), C.norm_weight(hd + 1, hd)
        t = dev(qkv)
        q = t[:, :nq * hd].view(T, nq, hd)
        k = t[:, nq * hd:(nq + nkv) * hd].view(T, nkv, hd)
        ops.qk_rmsnorm_rope(q, k, dev(qw), dev(kw), dev(ct), dev(st), positions=dev(pos), eps=1e-6)
        out = host(t)
        want_q = oracle.rmsnorm_rope(qkv[:, :nq * hd].reshape(T, nq, hd), qw, ct, st, pos, 1e-6)
        want_k = oracle.rmsnorm_rope(qkv[:, nq * hd:(nq + nkv) * hd].reshape(T, nkv, hd), kw, ct, st, pos, 1e-6)
        assert same(out[:, :nq * hd].reshape(T, nq, hd), want_q), (T, nq, nkv, hd, pad)
        assert same(out[:, nq * hd:(nq + nkv) * hd].reshape(T, nkv, hd), want_k), (T, nq, nkv, hd, pad)
        assert same(out[:, (nq + nkv) * hd:], qkv[:, (nq + nkv) * hd:]), (T, nq, nkv, hd, pad)


def test_sweep_swiglu_and_quantize(ops, oracle):
    def draw(r):
        return int(r.integers(1, 33)), int(r.integers(1, 5000)), int(r.choice([32, 64]))

    for rows, n, gs in shapes("swq", draw):
        g = C.normal(rows + n, (rows, n), 1.5)
        u = C.normal(rows + n + 1, (rows, n), 1.5)
        assert same(host(ops.swiglu(dev(g), dev(u))), oracle.swiglu(g, u)), ("swiglu", rows, n)
        wq, ws = oracle.swiglu_q8(g, u, gs)
        gq, gsc = ops.swiglu_q8(dev(g), dev(u), gs=gs)
        assert same(host(gq), wq) and same(host(gsc), ws), ("swiglu_q8", rows, n, gs)
        wq, ws = oracle.quantize(g, gs)
        gq, gsc = ops.quantize_q8(dev(g), gs=gs)
        assert same(host(gq), wq) and same(host(gsc), ws), ("quantize", rows, n, gs)


def test_sweep_embedding_and_kv_pack(ops, oracle):
    def draw(r):
        return int(r.integers(1, 3000)), 64 * int(r.integers(1, 97)), int(r.integers(1, 200))

    for vocab, dim, n in shapes("emb", draw):
        tq, ts = C.q8_table(vocab + dim, vocab, dim)
        ids = C.rng(n + vocab).integers(0, vocab, n).astype(np.int32)
        got = host(ops.embedding_gather_q8(dev(ids), dev(tq), dev(ts)))
        assert same(got, oracle.embedding_gather(ids, tq, ts, dim)), (vocab, dim, n)
        x = C.normal(n + dim, (n, dim), 8.0)
        h = host(ops.kv_pack_f16(dev(x))).view(np.uint16)
        assert same(h, oracle.kv_pack_f16(x)), ("kv_pack", n, dim)
        # K and V of fused rows [Q | K | V] (Q of a drawn width) in one launch
        kv = dim // 4 * 4 - 4 if dim > 64 else dim
        q_w = 4 * (dim % 13)
        qkv = C.normal(n + dim + 2, (n, q_w + 2 * kv), 8.0)
        d = dev(qkv)
        hk, hv = ops.kv_pack_f16_kv(d[:, q_w:q_w + kv], d[:, q_w + kv:])
        assert same(host(hk).view(np.uint16), oracle.kv_pack_f16(qkv[:, q_w:q_w + kv])), ("kv_pack K", n, kv, q_w)
        assert same(host(hv).view(np.uint16), oracle.kv_pack_f16(qkv[:, q_w + kv:])), ("kv_pack V", n, kv, q_w)


def test_sweep_embedding_many_tokens_with_invalid_ids(ops, oracle):
    """The gather at 1000-5000 tokens (many whole groups of 8 workgroups, then a bounds-tested last group; waves
    straddling rows wherever dim/4 is not a multiple of 64) with about 2% of the ids outside the table, whose
    rows must come out as zeros, wherever in a wave or piece they fall."""
    def draw(r):
        return int(r.integers(1, 5000)), 64 * int(r.integers(4, 33)), int(r.integers(1000, 5000))

    for vocab, dim, n in shapes("emb_many", draw):
        tq, ts = C.q8_table(vocab + dim + 1, vocab, dim)
        r = C.rng(n + vocab + 1)
        ids = r.integers(0, vocab, n).astype(np.int32)
        bad = r.random(n) < 0.02
        ids[bad] = np.where(r.random(int(bad.sum())) < 0.5, -1 - r.integers(0, 1000, int(bad.sum())),
                            vocab + r.integers(0, 1000, int(bad.sum()))).astype(np.int32)
        got = host(ops.embedding_gather_q8(dev(ids), dev(tq), dev(ts)))
        want = np.zeros((n, dim), np.float32)
        want[~bad] = oracle.embedding_gather(ids[~bad], tq, ts, dim)
        assert same(got, want), (vocab, dim, n, int(bad.sum()))


def test_sweep_qkv_stage(ops, oracle):
    """The Q/K/V stage with three sides: random head counts (partly filled waves), every head_dim class up to
    256, bias or not, norm or RoPE only, binary16 caches with or without the f32 result, random positions
    (token 0 at position 0: no rotation)."""
    def draw(r):
        return (int(r.integers(1, 24)), int(r.integers(1, 20)), int(r.integers(1, 9)), 32 * int(r.integers(2, 9)),
                bool(r.integers(0, 2)), bool(r.integers(0, 2)), bool(r.integers(0, 2)), bool(r.integers(0, 2)))

    for case in shapes("qkv", draw):
        qkv_case(ops, oracle, *case)


def test_sweep_qkv_stage_large(ops, oracle):
    """The same over 1024 to 2600 tokens (a quarter of the cases), where head counts that are not multiples of 8
    take the flat layout (8 (token, head) pairs of one side per wave, tokens in groups of 8)."""
    def draw(r):
        return (int(r.integers(1024, 2601)), int(r.integers(1, 20)), int(r.integers(1, 9)),
                32 * int(r.integers(2, 9)), bool(r.integers(0, 2)), bool(r.integers(0, 2)), bool(r.integers(0, 2)),
                bool(r.integers(0, 2)))

    for case in shapes("qkv_large", draw)[:max(1, CASES // 4)]:
        qkv_case(ops, oracle, *case)


def qkv_case(ops, oracle, T, nq, nkv, hd, norm, bias, keep_k, keep_v):
    case = (T, nq, nkv, hd, norm, bias, keep_k, keep_v)
    s = T * 31 + nq * 7 + nkv + hd
    qkv = C.normal(s, (T, (nq + 2 * nkv) * hd))
    qw, kw = C.norm_weight(s + 1, hd), C.norm_weight(s + 2, hd)
    qb = C.normal(s + 3, nq * hd, 0.5) if bias else None
    kb = C.normal(s + 4, nkv * hd, 0.5) if bias else None
    vb = C.normal(s + 5, nkv * hd, 0.5) if bias else None
    n_pos = T + 5
    ct, st = oracle.rope_tables(n_pos, hd, 1e6 if hd % 64 == 0 else 1e4)
    pos = C.rng(s + 6).integers(0, n_pos, T).astype(np.int32)
    pos[0] = 0
    q_np = qkv[:, :nq * hd].reshape(T, nq, hd)
    k_np = qkv[:, nq * hd:(nq + nkv) * hd].reshape(T, nkv, hd)
    v_np = qkv[:, (nq + nkv) * hd:].reshape(T, nkv, hd)
    wq, wk, wv, wkc, wvc = oracle.qkv_stage(q_np, k_np, v_np, qw if norm else None, kw if norm else None,
                                            qb, kb, vb, ct, st, pos, 1e-6)
    t = dev(qkv)
    q = t[:, :nq * hd].view(T, nq, hd)
    k = t[:, nq * hd:(nq + nkv) * hd].view(T, nkv, hd)
    v = t[:, (nq + nkv) * hd:].view(T, nkv, hd)
    kc = torch.zeros((T, nkv, hd), dtype=torch.float16, device="cuda")
    vc = torch.zeros((T, nkv, hd), dtype=torch.float16, device="cuda")
    d = lambda a: None if a is None else dev(a)  # noqa: E731
    ops.qkv_rope_stage(q, k, v, dev(ct), dev(st), positions=dev(pos), eps=1e-6,
                       q_norm_weight=d(qw) if norm else None, k_norm_weight=d(kw) if norm else None,
                       q_bias=d(qb), k_bias=d(kb), v_bias=d(vb), k_cache=kc, v_cache=vc, keep_k_f32=keep_k,
                       keep_v_f32=keep_v)
    out = host(t)
    assert same(out[:, :nq * hd].reshape(T, nq, hd), wq), ("q",) + case
    assert same(out[:, nq * hd:(nq + nkv) * hd].reshape(T, nkv, hd), wk if keep_k else k_np), ("k",) + case
    assert same(out[:, (nq + nkv) * hd:].reshape(T, nkv, hd), wv if keep_v else v_np), ("v",) + case
    assert same(host(kc).view(np.uint16), wkc), ("k cache",) + case
    assert same(host(vc).view(np.uint16), wvc), ("v cache",) + case
