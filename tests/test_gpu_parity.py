"""GPU parity: every kernel of libv7g.so against the CPU oracle on the same seeded inputs.

The bar is bit-exactness for every kernel: the oracle restates the reference
NASM kernels operation by operation, and the gfx950 kernels reproduce the same
operation order, so f32 outputs, int8 codes and scales compare with
np.array_equal (NaN positions compared as NaN).  The tolerances the
benchmark configurations allow (1e-5 relative for f32, +-1 code on 0.01% of
elements) are therefore not needed; the benchmark-size cases also report them.
"""
from __future__ import annotations

import numpy as np
import pytest

from tests import common as C

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def ops():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a visible MI355X")
    from v7multiplikator_amd import ops as _ops
    from v7multiplikator_amd import _lib
    _lib.load()
    return _ops


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def assert_bits(got, want, what=""):
    got = np.asarray(got)
    want = np.asarray(want)
    assert got.shape == want.shape, (what, got.shape, want.shape)
    if got.dtype.kind == "f":
        # +0/-0 must match too; a NaN matches any NaN (x86 makes its default NaN negative, the GPU positive)
        same = ((got == want) & (np.signbit(got) == np.signbit(want))) | (np.isnan(got) & np.isnan(want))
    else:
        same = got == want
    if not same.all():
        idx = np.argwhere(~same)[:5]
        raise AssertionError(f"{what}: {np.count_nonzero(~same)} of {got.size} differ; first {idx.tolist()} "
                             f"got {got[tuple(idx[0])]!r} want {want[tuple(idx[0])]!r}")


# --------------------------------------------------------------------------- arithmetic identities

def test_arith_selfcheck_exhaustive(ops):
    """rcp + Newton == 1/d, fma-corrected x/127 == IEEE x/127, the sigmoid with both == EVAL_SIGMOID with
    vdivps, and the binary16 conversion == round-to-nearest-even, each over its whole input range of binary32
    patterns on this device."""
    import ctypes

    from v7multiplikator_amd import _lib
    counts = (ctypes.c_ulonglong * 4)()
    rc = _lib.load().v7g_arith_selfcheck(ctypes.addressof(counts))
    assert rc == 0
    assert list(counts) == [0, 0, 0, 0]


# --------------------------------------------------------------------------- embedding gather (a9)

# Rows of 256 codes and wider run the flat-piece kernel: groups of 8 workgroups cover 8192 dwords (32768 codes)
# without a bounds test, a last group with one; a wave's 64 dwords may straddle two rows when dim/4 is not a
# multiple of 64 (320, 896, 1088, 1152).  Rows below 256 codes take one workgroup per row.
@pytest.mark.parametrize("vocab,dim,n", [(1000, 64, 7), (512, 128, 33), (1000, 192, 50), (800, 256, 3000),
                                         (1000, 320, 4099), (700, 896, 1001), (500, 1152, 517), (3000, 1024, 100),
                                         (4096, 4096, 257), (64, 4096, 1), (64, 4096, 2), (4096, 4096, 64),
                                         (700, 1088, 19), (900, 3072, 41), (600, 2048, 29), (500, 2560, 23),
                                         (400, 3584, 17), (300, 5120, 31), (200, 7168, 9), (300, 8192, 21),
                                         (100, 9216, 13)])
def test_embedding_gather_matches_oracle(ops, oracle, vocab, dim, n):
    tq, ts = C.q8_table(11, vocab, dim)
    ids = C.rng(12).integers(0, vocab, n).astype(np.int32)
    want = oracle.embedding_gather(ids, tq, ts, dim)
    got = ops.embedding_gather_q8(dev(ids), dev(tq), dev(ts))
    assert_bits(host(got), want, "embedding")


@pytest.mark.parametrize("dim", [128, 320, 896, 5120, 9216])
def test_embedding_invalid_ids_give_zero_rows(ops, oracle, dim):
    tq, ts = C.q8_table(3, 64, dim)
    ids = np.array([0, -1, 63, 64, 1 << 30, 5], np.int32)
    got = host(ops.embedding_gather_q8(dev(ids), dev(tq), dev(ts)))
    valid = np.array([0, 63, 5])
    want = oracle.embedding_gather(valid, tq, ts, dim)
    assert_bits(got[[0, 2, 5]], want, "valid rows")
    assert not got[[1, 3, 4]].any()


def test_embedding_empty(ops):
    tq, ts = C.q8_table(3, 16, 64)
    out = ops.embedding_gather_q8(torch.empty(0, dtype=torch.int32, device="cuda"), dev(tq), dev(ts))
    assert out.shape == (0, 64)


# --------------------------------------------------------------------------- fused add + RMSNorm (a1)

# The reference validator's sizes, tools/v_rmsnorm_validate.cpp:87-101, incl. leftover-block shapes.
@pytest.mark.parametrize("dim", [8, 16, 24, 48, 64, 128, 256, 1024, 2048, 3072, 8192, 40, 72, 16384])
@pytest.mark.parametrize("seed", [12345, 67890])
def test_fused_add_rmsnorm_validator_shapes(ops, oracle, dim, seed):
    rows = 5
    r = C.validator_row(seed, rows * dim).reshape(rows, dim)
    a = C.validator_row(seed + 1, rows * dim).reshape(rows, dim)
    w = C.validator_weight(seed + 2, dim)
    for eps in (1e-6, 1e-5):
        want_o, want_r = oracle.fused_add_rmsnorm(r, a, w, eps)
        rt = dev(r)
        got_o = ops.fused_add_rmsnorm(rt, dev(a), dev(w), eps=eps)
        assert_bits(host(rt), want_r, "residual")
        assert_bits(host(got_o), want_o, "o")


# Model widths: each compiled-in shape of the fixed-length row (2560, 3072, 3584, 3840, 5120, 8192), the run-time
# thread count with 1, 2 and 4 chunks per thread (1280, 1536 / 6144, 7168 / none below 8192 beyond those), the
# dispatch shapes (2048, 4096) and a multiple of 256 that falls back to the general kernel (4352); below 1024, the
# 256-thread row at the padded layout and, where the width is not a multiple of 32 (520, 776, 1000), at the natural
# one (more than 2048 such rows take one wave each: test_one_wave_rows).
MODEL_WIDTHS = [264, 320, 384, 512, 520, 576, 640, 768, 776, 896, 960, 1000,
                1280, 1536, 2048, 2560, 3072, 3584, 3840, 4096, 4352, 5120, 6144, 7168, 8192]


@pytest.mark.parametrize("dim", MODEL_WIDTHS)
def test_fused_add_rmsnorm_model_widths(ops, oracle, dim):
    rows = 37
    r = C.normal(dim, (rows, dim))
    a = C.normal(dim + 1, (rows, dim))
    w = C.norm_weight(dim + 2, dim)
    want_o, want_r = oracle.fused_add_rmsnorm(r, a, w, 1e-6)
    rt = dev(r)
    got_o = ops.fused_add_rmsnorm(rt, dev(a), dev(w), eps=1e-6)
    assert_bits(host(rt), want_r, f"residual dim={dim}")
    assert_bits(host(got_o), want_o, f"o dim={dim}")
    rt = dev(r)
    ops.fused_add_rmsnorm(rt, dev(a), dev(w), eps=1e-6, out=rt)
    assert_bits(host(rt), want_o, f"in-place o dim={dim}")


@pytest.mark.parametrize("dim", [264, 320, 448, 512, 520, 576, 640, 768, 776, 896, 960, 1000])
def test_one_wave_rows(ops, oracle, dim):
    """More than 2048 rows below 1024 floats: one wave per row with 2, 3 or 4 float4 chunks per lane, full (512,
    768) and partial, at the padded layout and the natural one (520, 776, 1000), through add+RMSNorm, RMSNorm,
    RMSNorm -> Q8 and its fused-add form (below 512: the 16-elements-per-thread quantizer starts at 512)."""
    rows = 2309
    r = C.normal(dim + 5, (rows, dim))
    a = C.normal(dim + 6, (rows, dim))
    w = C.norm_weight(dim + 7, dim)
    want_o, want_r = oracle.fused_add_rmsnorm(r, a, w, 1e-6)
    rt = dev(r)
    got_o = ops.fused_add_rmsnorm(rt, dev(a), dev(w), eps=1e-6)
    assert_bits(host(rt), want_r, f"residual dim={dim}")
    assert_bits(host(got_o), want_o, f"o dim={dim}")
    if dim % 32 == 0:
        assert_bits(host(ops.rmsnorm(dev(r), dev(w), eps=1e-5)), oracle.rmsnorm(r, w, 1e-5), f"rmsnorm dim={dim}")
    for gs in (32, 64):
        if dim % gs or dim >= 512:
            continue
        wq, ws = oracle.rmsnorm_quantize(r, w, 1e-6, gs)
        q, sc = ops.rmsnorm_quantize(dev(r), dev(w), eps=1e-6, gs=gs)
        assert_bits(host(q), wq, f"codes dim={dim} gs={gs}")
        assert_bits(host(sc), ws, f"scales dim={dim} gs={gs}")
        rt = dev(r)
        q, sc = ops.add_rmsnorm_quantize(rt, dev(a), dev(w), eps=1e-6, gs=gs)
        wq, ws = oracle.rmsnorm_quantize(want_r, w, 1e-6, gs)
        assert_bits(host(rt), want_r, f"add residual dim={dim} gs={gs}")
        assert_bits(host(q), wq, f"add codes dim={dim} gs={gs}")
        assert_bits(host(sc), ws, f"add scales dim={dim} gs={gs}")


def test_fused_add_rmsnorm_out_aliases_residual(ops, oracle):
    r = C.normal(5, (64, 2048))
    a = C.normal(6, (64, 2048))
    w = C.norm_weight(7, 2048)
    want_o, _ = oracle.fused_add_rmsnorm(r, a, w, 1e-6)
    rt = dev(r)
    ops.fused_add_rmsnorm(rt, dev(a), dev(w), eps=1e-6, out=rt)
    assert_bits(host(rt), want_o, "in-place o")


def test_fused_add_rmsnorm_config1(ops, oracle):
    """[512, 2048], x/residual ~N(0,1), w = 1+N(0,0.1), eps 1e-6."""
    r = C.normal(101, (512, 2048))
    a = C.normal(102, (512, 2048))
    w = C.norm_weight(103, 2048)
    want_o, want_r = oracle.fused_add_rmsnorm(r, a, w, 1e-6)
    rt = dev(r)
    got = ops.fused_add_rmsnorm(rt, dev(a), dev(w), eps=1e-6)
    assert_bits(host(rt), want_r, "residual")
    assert_bits(host(got), want_o, "o")


def test_fused_add_rmsnorm_empty(ops):
    w = torch.ones(64, device="cuda")
    r = torch.empty((0, 64), device="cuda")
    assert ops.fused_add_rmsnorm(r, r.clone(), w).shape == (0, 64)


# --------------------------------------------------------------------------- RMSNorm + RoPE (a3)

# tools/v_rmsnorm_validate.cpp:67-83: (heads, head_dim, pos, eps), tables theta 1e4, rope_max_dim = head_dim.
ROPE_VALIDATOR = [(1, 64, 0, 1e-6), (1, 64, 7, 1e-6), (4, 64, 0, 1e-6), (4, 64, 31, 1e-6), (8, 64, 7, 1e-6),
                  (8, 128, 0, 1e-6), (16, 64, 0, 1e-6), (16, 64, 31, 1e-6), (32, 64, 7, 1e-6), (32, 128, 0, 1e-6),
                  (40, 64, 31, 1e-6), (40, 128, 7, 1e-6), (32, 64, 0, 1e-5), (32, 64, 31, 1e-5), (8, 64, 7, 1e-5)]


@pytest.mark.parametrize("heads,hd,pos,eps", ROPE_VALIDATOR)
@pytest.mark.parametrize("seed", [12345, 67890])
def test_rmsnorm_rope_validator_cases(ops, oracle, heads, hd, pos, eps, seed):
    buf = C.validator_row(seed, heads * hd).reshape(1, heads, hd)
    w = C.validator_weight(seed + 1, hd)
    ct, st = C.validator_rope_tables(pos, hd, hd)
    want = oracle.rmsnorm_rope(buf, w, ct, st, np.array([pos], np.int32), eps)
    bt = dev(buf)
    ops.rmsnorm_rope_heads(bt, dev(w), dev(ct), dev(st), pos0=pos, eps=eps)
    assert_bits(host(bt), want, "rope")
    # the reference's own check: within 1e-3 of the double-precision C reference
    d = oracle.rmsnorm_rope_double_ref(buf, w, ct, st, [pos], eps)
    assert np.max(np.abs(host(bt) - d)) < 1e-3


@pytest.mark.parametrize("H", [3, 8])
@pytest.mark.parametrize("hd", [64, 96, 128, 160, 192, 224, 256, 288, 480, 512])
def test_rmsnorm_rope_head_dims(ops, oracle, hd, H):
    """Every head_dim % 32 == 0 in [64, 512] class: the wave kernel up to 224 (the rotate-half partner in the
    same lane, or for hd % 64 == 32 in lane m ^ 4), 16 lanes per head at 256 (the FMA chains handed between the
    two halves), the per-lane kernels above (register rotation for hd % 64 == 0, LDS rotation otherwise).
    37 tokens x 3 or 8 heads: partly filled waves, and with 8 heads the last workgroup's last waves hold no
    head."""
    T = 37
    buf = C.normal(hd, (T, H, hd))
    w = C.norm_weight(hd + 1, hd)
    ct, st = oracle.rope_tables(64, hd, 1e6)
    pos = C.rng(hd + 2).integers(0, 64, T).astype(np.int32)
    pos[0] = 0
    want = oracle.rmsnorm_rope(buf, w, ct, st, pos, 1e-6)
    bt = dev(buf)
    ops.rmsnorm_rope_heads(bt, dev(w), dev(ct), dev(st), positions=dev(pos), eps=1e-6)
    assert_bits(host(bt), want, f"rope hd={hd} H={H}")


def test_qk_rmsnorm_rope_config2(ops, oracle):
    """T=2048, 16 Q + 8 KV heads, hd 128, theta 1e6, positions 0..T-1, inside a fused QKV row."""
    T, Hq, Hk, D = 2048, 16, 8, 128
    qkv = C.normal(201, (T, (Hq + 2 * Hk) * D))
    qw = C.norm_weight(202, D)
    kw = C.norm_weight(203, D)
    ct, st = oracle.rope_tables(T, D, 1e6)
    pos = np.arange(T, dtype=np.int32)
    q_np = qkv[:, :Hq * D].reshape(T, Hq, D)
    k_np = qkv[:, Hq * D:(Hq + Hk) * D].reshape(T, Hk, D)
    want_q = oracle.rmsnorm_rope(q_np, qw, ct, st, pos, 1e-6)
    want_k = oracle.rmsnorm_rope(k_np, kw, ct, st, pos, 1e-6)
    t = dev(qkv)
    q = t[:, :Hq * D].view(T, Hq, D)
    k = t[:, Hq * D:(Hq + Hk) * D].view(T, Hk, D)
    ops.qk_rmsnorm_rope(q, k, dev(qw), dev(kw), dev(ct), dev(st), positions=dev(pos), eps=1e-6)
    out = host(t)
    assert_bits(out[:, :Hq * D].reshape(T, Hq, D), want_q, "q")
    assert_bits(out[:, Hq * D:(Hq + Hk) * D].reshape(T, Hk, D), want_k, "k")
    assert_bits(out[:, (Hq + Hk) * D:], qkv[:, (Hq + Hk) * D:], "v untouched")


@pytest.mark.parametrize("Hq,Hk,D", [(28, 4, 128), (14, 2, 64), (12, 2, 64), (20, 6, 64), (32, 17, 64), (40, 8, 96),
                                     (17, 1, 96), (16, 8, 256), (10, 3, 256), (5, 1, 256)])
def test_qk_rmsnorm_rope_partial_waves(ops, oracle, Hq, Hk, D):
    """Head counts that are not multiples of a wave's heads (Qwen2.5-style 28 + 4, and 14 + 2 up to 40 + 8 at
    head_dim 64 and 96, at 8 heads per wave; 10 + 3 and 5 + 1 at head_dim 256, 4 heads per wave of 16 lanes each):
    the last wave of each side holds fewer heads; its spare lanes must store nothing."""
    T = 37
    qkv = C.normal(Hq * 100 + Hk, (T, (Hq + 2 * Hk) * D))
    qw, kw = C.norm_weight(Hq + 1, D), C.norm_weight(Hk + 2, D)
    ct, st = oracle.rope_tables(64, D, 1e6)
    pos = C.rng(Hq).integers(0, 64, T).astype(np.int32)
    pos[5] = 0
    q_np = qkv[:, :Hq * D].reshape(T, Hq, D)
    k_np = qkv[:, Hq * D:(Hq + Hk) * D].reshape(T, Hk, D)
    t = dev(qkv)
    q = t[:, :Hq * D].view(T, Hq, D)
    k = t[:, Hq * D:(Hq + Hk) * D].view(T, Hk, D)
    ops.qk_rmsnorm_rope(q, k, dev(qw), dev(kw), dev(ct), dev(st), positions=dev(pos), eps=1e-6)
    out = host(t)
    assert_bits(out[:, :Hq * D].reshape(T, Hq, D), oracle.rmsnorm_rope(q_np, qw, ct, st, pos, 1e-6), "q")
    assert_bits(out[:, Hq * D:(Hq + Hk) * D].reshape(T, Hk, D), oracle.rmsnorm_rope(k_np, kw, ct, st, pos, 1e-6), "k")
    assert_bits(out[:, (Hq + Hk) * D:], qkv[:, (Hq + Hk) * D:], "v untouched")


@pytest.mark.parametrize("T,nq,nkv,hd,norm,bias,keep_k,keep_v,pos0", [
    (2049, 14, 2, 64, False, True, True, True, None),     # Qwen2.5-0.5B: bias through the weight registers
    (1024, 12, 2, 128, False, True, False, True, None),   # Qwen2.5-1.5B at 1024 tokens (half the lanes would idle)
    (2048, 28, 4, 128, True, True, True, False, None),    # norm weight and bias on one side
    (2055, 7, 1, 96, True, False, True, True, 5),         # odd head_dim / 32, positions pos0 + t
    (2050, 3, 3, 160, False, False, True, True, None),
    (2051, 12, 4, 192, False, True, True, True, None),
    (2053, 5, 2, 224, True, True, False, False, None),
    (2049, 4, 1, 256, True, False, True, True, None),     # Gemma-3-1B: 16 lanes per head, 4 pairs per wave
    (1030, 1, 1, 256, False, True, True, False, None),
    (2051, 6, 3, 256, True, True, False, True, 7)])
def test_qkv_stage_flat_layout(ops, oracle, T, nq, nkv, hd, norm, bias, keep_k, keep_v, pos0):
    """From 1024 or 2048 tokens, head counts that are not multiples of a wave's heads take the flat layout (8
    (token, head) pairs of one side per wave over groups of 8 tokens, 4 over groups of 4 at head_dim 256; each lane
    group with its own position): last groups of fewer tokens, positions 0 (no rotation) and past the tables (NaN
    in Q and K, V kept), every head_dim / 32 from 2 to 8, bias or norm weight or both, cache rows with and without
    the f32 result."""
    s = T + 7 * nq + hd
    qkv = C.normal(s, (T, (nq + 2 * nkv) * hd))
    qw, kw = C.norm_weight(s + 1, hd), C.norm_weight(s + 2, hd)
    qb = C.normal(s + 3, nq * hd, 0.5) if bias else None
    kb = C.normal(s + 4, nkv * hd, 0.5) if bias else None
    vb = C.normal(s + 5, nkv * hd, 0.5) if bias else None
    n_pos = 3000
    ct, st = oracle.rope_tables(n_pos, hd, 1e6 if hd % 64 == 0 else 1e4)
    bad = np.array([], np.int64)
    if pos0 is None:
        pos = C.rng(s + 6).integers(0, n_pos, T).astype(np.int32)
        pos[[0, 9, T - 1]] = 0
        bad = np.array([3, 17, T - 2])
        pos[bad] = [n_pos, n_pos + 100, 2 ** 31 - 1]
    else:
        pos = (np.arange(T) + pos0).astype(np.int32)
    q_np = qkv[:, :nq * hd].reshape(T, nq, hd)
    k_np = qkv[:, nq * hd:(nq + nkv) * hd].reshape(T, nkv, hd)
    v_np = qkv[:, (nq + nkv) * hd:].reshape(T, nkv, hd)
    opos = pos.copy()
    opos[bad] = 0  # the oracle's tables have no such rows; these tokens are checked for NaN below
    wq, wk, wv, wkc, wvc = oracle.qkv_stage(q_np, k_np, v_np, qw if norm else None, kw if norm else None, qb, kb, vb,
                                            ct, st, opos, 1e-6)
    t = dev(qkv)
    q = t[:, :nq * hd].view(T, nq, hd)
    k = t[:, nq * hd:(nq + nkv) * hd].view(T, nkv, hd)
    v = t[:, (nq + nkv) * hd:].view(T, nkv, hd)
    kc = torch.zeros((T, nkv, hd), dtype=torch.float16, device="cuda")
    vc = torch.zeros((T, nkv, hd), dtype=torch.float16, device="cuda")
    d = lambda a: None if a is None else dev(a)  # noqa: E731
    ops.qkv_rope_stage(q, k, v, dev(ct), dev(st), positions=None if pos0 is not None else dev(pos),
                       pos0=pos0 or 0, eps=1e-6, q_norm_weight=d(qw) if norm else None,
                       k_norm_weight=d(kw) if norm else None, q_bias=d(qb), k_bias=d(kb), v_bias=d(vb), k_cache=kc,
                       v_cache=vc, keep_k_f32=keep_k, keep_v_f32=keep_v)
    out = host(t)
    gq = out[:, :nq * hd].reshape(T, nq, hd)
    gk = out[:, nq * hd:(nq + nkv) * hd].reshape(T, nkv, hd)
    gv = out[:, (nq + nkv) * hd:].reshape(T, nkv, hd)
    gkc, gvc = host(kc), host(vc)
    ok = np.setdiff1d(np.arange(T), bad)
    assert_bits(gq[ok], wq[ok], "q")
    assert_bits(gk[ok], (wk if keep_k else k_np)[ok], "k")
    assert_bits(gv, wv if keep_v else v_np, "v")
    assert_bits(gkc.view(np.uint16)[ok], wkc[ok], "k cache")
    assert_bits(gvc.view(np.uint16), wvc, "v cache")
    assert np.isnan(gq[bad]).all() and np.isnan(gkc[bad].astype(np.float32)).all()
    if keep_k:
        assert np.isnan(gk[bad]).all()


@pytest.mark.parametrize("T,H,hd", [(2050, 3, 64), (2049, 5, 96), (2051, 12, 128), (2053, 3, 256), (1027, 1, 160)])
def test_single_side_entries_in_the_flat_layout(ops, oracle, T, H, hd):
    """v7g_rmsnorm_rope_heads and v7g_rope_only_heads over one side whose head count is not a multiple of a
    wave's heads, from 1024 tokens: the flat layout with a single side (token stride wider than the heads)."""
    stride = H * hd + 64
    buf = C.normal(T + H + hd, (T, stride))
    w = C.norm_weight(hd + 11, hd)
    ct, st = oracle.rope_tables(T + 1, hd, 1e6 if hd % 64 == 0 else 1e4)
    pos = C.rng(T + hd).integers(0, T + 1, T).astype(np.int32)
    pos[[1, T - 1]] = 0
    heads = buf[:, :H * hd].reshape(T, H, hd)
    bt = dev(buf)
    ops.rmsnorm_rope_heads(bt[:, :H * hd].view(T, H, hd), dev(w), dev(ct), dev(st), positions=dev(pos), eps=1e-6)
    got = host(bt)
    assert_bits(got[:, :H * hd].reshape(T, H, hd), oracle.rmsnorm_rope(heads, w, ct, st, pos, 1e-6), "rmsnorm_rope")
    assert_bits(got[:, H * hd:], buf[:, H * hd:], "gap untouched")
    bt = dev(buf)
    ops.rope_only_heads(bt[:, :H * hd].view(T, H, hd), dev(ct), dev(st), positions=dev(pos))
    assert_bits(host(bt)[:, :H * hd].reshape(T, H, hd), oracle.rope_only(heads, ct, st, pos), "rope only")


@pytest.mark.parametrize("H", [2, 8])
def test_rope_position_outside_tables_gives_nan(ops, oracle, H):
    buf = C.normal(9, (3, H, 64))
    w = C.norm_weight(10, 64)
    ct, st = oracle.rope_tables(8, 64, 1e4)
    pos = np.array([3, 8, 0], np.int32)  # 8 is past the 8-row tables
    bt = dev(buf)
    ops.rmsnorm_rope_heads(bt, dev(w), dev(ct), dev(st), positions=dev(pos))
    got = host(bt)
    want = oracle.rmsnorm_rope(buf[[0, 2]], w, ct, st, pos[[0, 2]], 1e-6)
    assert_bits(got[[0, 2]], want, "valid tokens")
    assert np.isnan(got[1]).all()


@pytest.mark.parametrize("head_dim,base", [(128, 1e6), (64, 1e4), (256, 5e6)])
def test_rope_tables_builder(ops, oracle, head_dim, base):
    """The library's host builder runs the reference's x87 sequence (fyl2x/f2xm1/fscale frequencies, fsincos):
    its tables equal the oracle's bit for bit."""
    c, s = ops.rope_tables(4096, head_dim, base)
    wc, ws = oracle.rope_tables(4096, head_dim, base)
    assert_bits(host(c), wc, "cos")
    assert_bits(host(s), ws, "sin")


# --------------------------------------------------------------------------- SwiGLU (a5, a6)

SPECIAL = np.array([0.0, -0.0, 1.0, -1.0, 80.0, -80.0, 80.5, -80.5, 100.0, -100.0, 1e-30, -1e-30, 3e38, -3e38,
                    np.inf, -np.inf, np.nan, 0.5, 88.7, -88.7, 1e-45, 2.0 ** -126], np.float32)


def test_swiglu_special_values(ops, oracle):
    g = np.repeat(SPECIAL, SPECIAL.size)
    u = np.tile(SPECIAL, SPECIAL.size)
    want = oracle.swiglu(g, u)
    got = ops.swiglu(dev(g), dev(u))
    assert_bits(host(got), want, "swiglu special")


@pytest.mark.parametrize("n", [1, 3, 4, 5, 1023, 4096, 100003])
def test_swiglu_lengths(ops, oracle, n):
    g = C.normal(n, n, 1.5)
    u = C.normal(n + 1, n, 1.5)
    assert_bits(host(ops.swiglu(dev(g), dev(u))), oracle.swiglu(g, u), "swiglu")


def test_swiglu_config3_and_in_place(ops, oracle):
    """gate, up [4096, 6144] ~N(0, 1.5); also in place over gate as .pq_ffn_silu does."""
    g = C.normal(301, (4096, 6144), 1.5)
    u = C.normal(302, (4096, 6144), 1.5)
    want = oracle.swiglu(g, u)
    gt = dev(g)
    ops.swiglu(gt, dev(u), out=gt)
    got = host(gt)
    assert_bits(got, want, "swiglu config3")
    ref = (g.astype(np.float64) / (1.0 + np.exp(-g.astype(np.float64)))) * u
    rel = np.abs(got - ref) / np.maximum(np.abs(ref), 1e-30)
    assert np.max(rel[np.abs(ref) > 1e-30]) < 1e-5


# --------------------------------------------------------------------------- quantize (a7) and SwiGLU->Q8 (a8)

@pytest.mark.parametrize("pattern", C.KT_PATTERNS)
@pytest.mark.parametrize("n", [64, 256, 1024, 4096, 8192, 65536])
@pytest.mark.parametrize("gs", [64, 32])
def test_quantize_validator_patterns(ops, oracle, pattern, n, gs):
    for seed in (12345, 67890, 11111):
        x = C.kt_pattern(pattern, n, seed)
        wq, ws = oracle.quantize(x[None], gs)
        gq, gsc = ops.quantize_q8(dev(x[None]), gs=gs)
        assert_bits(host(gq), wq, f"codes {pattern}")
        assert_bits(host(gsc), ws, f"scales {pattern}")
        if gs == 64:
            kq, _ = oracle.kt_quantize_c_ref(x)
            assert_bits(host(gq)[0], kq, "codes vs kt_quantize_c_ref")


@pytest.mark.parametrize("rows,row_len,gs", [(1, 100, 64), (3, 1000, 64), (7, 65, 32), (2, 3, 64), (5, 130, 32),
                                             (4, 8192, 64), (3, 257, 16)])
def test_quantize_tails_and_ragged(ops, oracle, rows, row_len, gs):
    x = C.normal(rows * row_len, (rows, row_len), 3.0)
    wq, ws = oracle.quantize(x, gs)
    gq, gsc = ops.quantize_q8(dev(x), gs=gs)
    assert_bits(host(gq), wq, "codes")
    assert_bits(host(gsc), ws, "scales")


def test_quantize_non_finite(ops, oracle):
    x = C.normal(1, (4, 64))
    x[0, 5] = np.inf
    x[2, 63] = np.nan
    x[3, :] = 0.0
    wq, ws = oracle.quantize(x, 64)
    gq, gsc = ops.quantize_q8(dev(x), gs=64)
    # an Inf row gives scale Inf, codes 0 and -127; the NaN at element 63 reaches the group max through
    # the reference's vmaxps tree, which the floor then replaces (scale 2^-126, every code -127)
    assert_bits(host(gq), wq, "codes")
    assert_bits(host(gsc), ws, "scales")
    assert host(gsc)[2, 0] == np.float32(2.0 ** -126) and np.all(host(gq)[2] == -127)


def nan_groups(seed, rows, row_len, gs):
    """Rows of groups where a NaN sits at every position of the group in turn, beside a large value
    (2^40, which a NaN can take out of the group max) and tiny ones (which the floor scale turns into
    codes from 0 to -127 past 2^31); a third of the rows carry many NaN at random positions."""
    x = C.normal(seed, (rows, row_len), 1.0)
    rng = C.rng(seed + 1)
    for r in range(rows):
        for g0 in range(0, row_len - gs + 1, gs):
            p = (r + g0 // gs) % gs
            x[r, g0 + p] = np.nan
            x[r, g0 + (p * 7 + 3 + r // gs) % gs] = np.float32(2.0 ** 40) * (1 - 2 * (r & 1))
            x[r, g0 + (p + 1) % gs] = np.float32(3 * 2.0 ** -126)
            x[r, g0 + (p + 2) % gs] = np.float32(2.0 ** -94)
        if r % 3 == 2:
            x[r, rng.integers(0, row_len, max(row_len // 8, 1))] = np.nan
    return x


@pytest.mark.parametrize("rows,row_len,gs", [(128, 128, 64), (64, 96, 32), (96, 1000, 64), (40, 1000, 32),
                                             (16, 257, 16)])
def test_quantize_nan_groups_follow_the_reference_tree(ops, oracle, rows, row_len, gs):
    """A NaN in a group: the reference's vmaxps tree (src/asm/quantize_kernel.inc:62-84) lets it reach the
    group max or drop out, with the values it was paired with, depending on its position.  Flat groups
    (row_len a multiple of gs), groups of the general path (ragged rows) and their scalar tails, bit for bit."""
    x = nan_groups(rows * row_len + gs, rows, row_len, gs)
    wq, ws = oracle.quantize(x, gs)
    gq, gsc = ops.quantize_q8(dev(x), gs=gs)
    assert_bits(host(gq), wq, "codes")
    assert_bits(host(gsc), ws, "scales")


@pytest.mark.parametrize("gs", [32, 64])
def test_swiglu_q8_nan_groups(ops, oracle, gs):
    g = nan_groups(77 + gs, 64, 4096, gs)
    u = C.normal(78 + gs, (64, 4096), 1.5)
    u[5, 100:140] = np.nan
    wq, ws = oracle.swiglu_q8(g, u, gs)
    gq, gsc = ops.swiglu_q8(dev(g), dev(u), gs=gs)
    assert_bits(host(gq), wq, "codes")
    assert_bits(host(gsc), ws, "scales")


@pytest.mark.parametrize("gs", [32, 64])
def test_rmsnorm_quantize_nan_columns(ops, oracle, gs):
    """NaN weights put a NaN at the same column of every row (the row's scale is unaffected), one NaN input
    makes its whole row NaN: both follow the reference's tree (src/asm/rmsnorm_quantize_kernel.inc:158-187)."""
    dim, rows = 2048, 2 * gs
    x = C.normal(91, (rows, dim))
    x[3, 17] = np.nan
    w = C.norm_weight(92, dim)
    w[np.arange(0, dim, dim // 32) + np.arange(32) % gs] = np.nan
    wq, ws = oracle.rmsnorm_quantize(x, w, 1e-6, gs)
    q, s = ops.rmsnorm_quantize(dev(x), dev(w), eps=1e-6, gs=gs)
    assert_bits(host(q), wq, "codes")
    assert_bits(host(s), ws, "scales")
    r = C.normal(93, (rows, dim))
    a = C.normal(94, (rows, dim))
    wq, ws = oracle.rmsnorm_quantize(oracle.add_inplace(r, a), w, 1e-6, gs)
    q, s = ops.add_rmsnorm_quantize(dev(r), dev(a), dev(w), eps=1e-6, gs=gs)
    assert_bits(host(q), wq, "codes")
    assert_bits(host(s), ws, "scales")


@pytest.mark.parametrize("gs", [32, 64])
@pytest.mark.parametrize("dim", [544, 4096, 12288])
def test_rmsnorm_quantize_nan_at_every_group_position(ops, oracle, gs, dim):
    """A NaN weight at each position of a quantization group in turn (group g: position g % gs), beside a
    weight of 2^20 two positions on, through the 16-elements-per-thread kernel (dims 544: a partial wave of
    34 threads, GS 32 only; 4096; 12288): the reference's ordered vmaxps tree keeps the NaN or drops it with
    its partners (src/asm/rmsnorm_quantize_kernel.inc:158-187).  Also with the residual add fused in front."""
    if dim % gs:
        pytest.skip("dim must be a multiple of the group size")
    rows = 3
    groups = dim // gs
    x = C.normal(95 + dim, (rows, dim))
    w = C.norm_weight(96 + dim, dim)
    g = np.arange(groups)
    w[g * gs + g % gs] = np.nan
    w[g * gs + (g + 2) % gs] = np.float32(2.0 ** 20)
    wq, ws = oracle.rmsnorm_quantize(x, w, 1e-6, gs)
    q, s = ops.rmsnorm_quantize(dev(x), dev(w), eps=1e-6, gs=gs)
    assert_bits(host(q), wq, "codes")
    assert_bits(host(s), ws, "scales")
    r = C.normal(97 + dim, (rows, dim))
    a = C.normal(98 + dim, (rows, dim))
    r_new = oracle.add_inplace(r, a)
    wq, ws = oracle.rmsnorm_quantize(r_new, w, 1e-6, gs)
    rt = dev(r)
    q, s = ops.add_rmsnorm_quantize(rt, dev(a), dev(w), eps=1e-6, gs=gs)
    assert_bits(host(rt), r_new, "residual")
    assert_bits(host(q), wq, "fused codes")
    assert_bits(host(s), ws, "fused scales")


@pytest.mark.parametrize("gs", [32, 64])
@pytest.mark.parametrize("rows,hidden", [(1, 64), (3, 192), (16, 8192), (5, 96)])
def test_swiglu_q8_shapes(ops, oracle, gs, rows, hidden):
    # hidden 96 with gs 64: each row ends in a 32-element tail group, quantized on its own as the
    # reference's scalar tail does (src/asm/quantize_kernel.inc:119-152)
    g = C.normal(rows + hidden, (rows, hidden), 1.5)
    u = C.normal(rows + hidden + 1, (rows, hidden), 1.5)
    wq, ws = oracle.swiglu_q8(g, u, gs)
    gq, gsc = ops.swiglu_q8(dev(g), dev(u), gs=gs)
    assert_bits(host(gq), wq, "codes")
    assert_bits(host(gsc), ws, "scales")


def test_swiglu_q8_config4(ops, oracle):
    """gate, up [4096, 8192] ~N(0, 1.5), 32-element blocks."""
    g = C.normal(401, (4096, 8192), 1.5)
    u = C.normal(402, (4096, 8192), 1.5)
    wq, ws = oracle.swiglu_q8(g, u, 32)
    gq, gsc = ops.swiglu_q8(dev(g), dev(u), gs=32)
    assert_bits(host(gq), wq, "codes")
    assert_bits(host(gsc), ws, "scales")


# --------------------------------------------------------------------------- rmsnorm, rmsnorm_quantize, add_inplace

@pytest.mark.parametrize("dim", [64, 128, 256, 1024, 2048, 3072, 4096, 8192, 16384])
@pytest.mark.parametrize("seed", [12345, 67890])
def test_rmsnorm_rows(ops, oracle, dim, seed):
    rows = 5
    x = C.validator_row(seed, rows * dim).reshape(rows, dim)
    w = C.validator_weight(seed + 1, dim)
    for eps in (1e-6, 1e-5):
        got = ops.rmsnorm(dev(x), dev(w), eps=eps)
        assert_bits(host(got), oracle.rmsnorm(x, w, eps), f"rmsnorm dim={dim}")
    xt = dev(x)
    ops.rmsnorm(xt, dev(w), out=xt)  # in place
    assert_bits(host(xt), oracle.rmsnorm(x, w, 1e-6), "rmsnorm in place")


@pytest.mark.parametrize("dim", MODEL_WIDTHS)
def test_rmsnorm_model_widths(ops, oracle, dim):
    if dim % 32:
        pytest.skip("RMSNorm takes whole 32-float blocks")
    rows = 37
    x = C.normal(dim + 3, (rows, dim), 2.0)
    w = C.norm_weight(dim + 4, dim)
    want = oracle.rmsnorm(x, w, 1e-5)
    assert_bits(host(ops.rmsnorm(dev(x), dev(w), eps=1e-5)), want, f"rmsnorm dim={dim}")
    xt = dev(x)
    ops.rmsnorm(xt, dev(w), eps=1e-5, out=xt)
    assert_bits(host(xt), want, f"rmsnorm in place dim={dim}")


@pytest.mark.parametrize("gs", [64, 32])
@pytest.mark.parametrize("dim", [64, 128, 192, 320, 384, 448, 512, 544, 1024, 2048, 2560, 3072, 3584, 3840, 4096,
                                 5120, 6144, 7168, 8192, 12288, 16384])
def test_rmsnorm_quantize_rows(ops, oracle, gs, dim):
    if dim % gs:
        pytest.skip("dim must be a multiple of the group size")
    rows = 7
    x = C.normal(dim + gs, (rows, dim))
    w = C.norm_weight(dim, dim)
    wq, ws = oracle.rmsnorm_quantize(x, w, 1e-6, gs)
    q, s = ops.rmsnorm_quantize(dev(x), dev(w), eps=1e-6, gs=gs)
    assert_bits(host(q), wq, "codes")
    assert_bits(host(s), ws, "scales")


@pytest.mark.parametrize("gs", [64, 32])
@pytest.mark.parametrize("dim", [64, 320, 448, 2048, 2560, 3072, 3584, 3840, 4096, 5120, 6144, 8192, 12288])
def test_add_rmsnorm_quantize_equals_the_two_calls(ops, oracle, gs, dim):
    """The fused decode step equals v7s_add_inplace then v7s_rmsnorm_quantize (src/asm/forward_q8.inc:386-387)."""
    rows = 9
    r = C.normal(dim, (rows, dim))
    a = C.normal(dim + 1, (rows, dim))
    w = C.norm_weight(dim + 2, dim)
    r_new = oracle.add_inplace(r, a)
    wq, ws = oracle.rmsnorm_quantize(r_new, w, 1e-6, gs)
    rt = dev(r)
    q, s = ops.add_rmsnorm_quantize(rt, dev(a), dev(w), eps=1e-6, gs=gs)
    assert_bits(host(rt), r_new, "residual")
    assert_bits(host(q), wq, "codes")
    assert_bits(host(s), ws, "scales")


@pytest.mark.parametrize("gs", [64, 32])
@pytest.mark.parametrize("rows,dim", [(64, 4096), (2309, 768)])
@pytest.mark.parametrize("fused_add", [False, True])
def test_rmsnorm_quantize_codes_4_byte_aligned(ops, oracle, gs, rows, dim, fused_add):
    """Codes that are 4-byte but not 16-byte aligned (the C ABI accepts them) send dims 512..12288 to the row
    kernel's 4-elements-per-lane quantizer instead of the 16-per-thread kernel: [64, 4096] runs the 256-thread
    row, [2309, 768] (more than 2048 rows) the one-wave row.  Through the C ABI, plain and with the fused add,
    bit-exact against the oracle; the bytes around the codes stay untouched."""
    import ctypes

    from v7multiplikator_amd import _lib
    L = _lib.load()
    x = C.normal(rows + dim + gs, (rows, dim))
    a = C.normal(rows + dim + gs + 1, (rows, dim))
    w = C.norm_weight(dim + gs, dim)
    n = rows * dim
    qbuf = torch.full((n + 32,), 77, dtype=torch.int8, device="cuda")
    q_ptr = qbuf.data_ptr() + 4
    assert q_ptr % 16 == 4
    st = torch.empty((rows, dim // gs), dtype=torch.float32, device="cuda")
    xt, at, wt = dev(x), dev(a), dev(w)
    ops._bind(xt)
    if fused_add:
        rc = L.v7g_add_rmsnorm_quantize(q_ptr, st.data_ptr(), xt.data_ptr(), at.data_ptr(), wt.data_ptr(), rows, dim,
                                        gs, ctypes.c_float(1e-6))
        x = oracle.add_inplace(x, a)
    else:
        rc = L.v7g_rmsnorm_quantize(q_ptr, st.data_ptr(), xt.data_ptr(), wt.data_ptr(), rows, dim, gs,
                                    ctypes.c_float(1e-6))
    assert rc == 0
    torch.cuda.synchronize()
    wq, ws = oracle.rmsnorm_quantize(x, w, 1e-6, gs)
    got = host(qbuf)
    assert_bits(got[4:4 + n].reshape(rows, dim), wq, "codes")
    assert_bits(host(st), ws, "scales")
    assert (got[:4] == 77).all() and (got[4 + n:] == 77).all()
    if fused_add:
        assert_bits(host(xt), x, "residual")


def test_rmsnorm_quantize_config_shape(ops, oracle):
    """The Q8 path's per-token input to QKV/W1/W3 at the Qwen3-8B width: [2048, 4096], GS 64."""
    x = C.normal(11, (2048, 4096))
    w = C.norm_weight(12, 4096)
    wq, ws = oracle.rmsnorm_quantize(x, w, 1e-6, 64)
    q, s = ops.rmsnorm_quantize(dev(x), dev(w), eps=1e-6, gs=64)
    assert_bits(host(q), wq, "codes")
    assert_bits(host(s), ws, "scales")


@pytest.mark.parametrize("n", [1, 3, 32, 96, 160, 1024, 2048, 100003])
def test_add_inplace(ops, oracle, n):
    x = C.normal(n, n)
    y = C.normal(n + 1, n)
    xt = dev(x)
    ops.add_inplace(xt, dev(y))
    assert_bits(host(xt), oracle.add_inplace(x, y), "add_inplace")


# --------------------------------------------------------------------------- v7s_kv_pack_f16, fused K pack

F16_SPECIAL = np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 65519.99, 65520.0, -65520.0, 1e30, -1e30, 2.0 ** -24,
                        2.0 ** -25, 3 * 2.0 ** -26, 2.0 ** -14 - 2.0 ** -25, 1e-30, np.inf, -np.inf, 0.1, 1 / 3.0,
                        2049.0, 2051.0, 4097.5, -7.0e-6, 6.1e-5], np.float32)


def test_kv_pack_f16_special_values(ops, oracle):
    x = np.concatenate([F16_SPECIAL, np.zeros(8 - F16_SPECIAL.size % 8, np.float32)]).reshape(1, -1)
    got = host(ops.kv_pack_f16(dev(x))).view(np.uint16)
    assert_bits(got, oracle.kv_pack_f16(x), "special")
    xn = np.full((1, 8), np.nan, np.float32)
    gn = host(ops.kv_pack_f16(dev(xn))).view(np.uint16)
    assert np.all((gn & 0x7C00) == 0x7C00) and np.all(gn & 0x03FF)


@pytest.mark.parametrize("rows,row_len,src_stride,dst_stride", [(1, 8, 8, 8), (5, 1024, 1024, 1024),
                                                                (37, 1024, 6144, 1024), (8192, 1024, 6144, 2048)])
def test_kv_pack_f16_rows_strided(ops, oracle, rows, row_len, src_stride, dst_stride):
    """K or V rows out of a fused QKV row [Q | K | V] into cache rows (strides in elements)."""
    src = C.normal(rows + row_len, (rows, src_stride), 2.0)
    st = dev(src)
    cache = torch.zeros((rows, dst_stride), dtype=torch.float16, device="cuda")
    ops.kv_pack_f16(st[:, :row_len], out=cache[:, :row_len])
    got = host(cache).view(np.uint16)
    assert_bits(got[:, :row_len], oracle.kv_pack_f16(src[:, :row_len]), "packed rows")
    assert not got[:, row_len:].any()


@pytest.mark.parametrize("rows,kv_dim,q_dim,cache_stride", [(1, 8, 32, 8), (37, 1024, 4096, 1024),
                                                             (8192, 1024, 4096, 1024), (9, 1284, 2048, 1300),
                                                             (3, 4100, 0, 4104)])
def test_kv_pack_f16_kv_one_launch(ops, oracle, rows, kv_dim, q_dim, cache_stride):
    """K and V rows of fused QKV rows [Q | K | V] into two binary16 caches in one launch, each equal to its own
    v7s_kv_pack_f16 (rows of 1284 and 4100 floats: partial last blocks, more than one block per row)."""
    qkv = C.normal(rows + kv_dim, (rows, q_dim + 2 * kv_dim), 2.0)
    d = dev(qkv)
    kc = torch.zeros((rows, cache_stride), dtype=torch.float16, device="cuda")
    vc = torch.zeros((rows, cache_stride), dtype=torch.float16, device="cuda")
    ops.kv_pack_f16_kv(d[:, q_dim:q_dim + kv_dim], d[:, q_dim + kv_dim:], k_out=kc[:, :kv_dim], v_out=vc[:, :kv_dim])
    k = host(kc).view(np.uint16)
    v = host(vc).view(np.uint16)
    assert_bits(k[:, :kv_dim], oracle.kv_pack_f16(qkv[:, q_dim:q_dim + kv_dim]), "K rows")
    assert_bits(v[:, :kv_dim], oracle.kv_pack_f16(qkv[:, q_dim + kv_dim:]), "V rows")
    assert not k[:, kv_dim:].any() and not v[:, kv_dim:].any()
    assert np.array_equal(host(d), qkv)


@pytest.mark.parametrize("heads", [(8, 2), (16, 8)])
@pytest.mark.parametrize("keep", [True, False])
@pytest.mark.parametrize("hd", [128, 96])
def test_qk_rope_with_fused_k_pack(ops, oracle, keep, hd, heads):
    """RMSNorm+RoPE of Q and K plus the binary16 K cache rows in one launch == RoPE, then v7s_kv_pack_f16 of K."""
    T = 67
    Hq, Hk = heads
    qkv = C.normal(hd + 5, (T, (Hq + 2 * Hk) * hd))
    qw = C.norm_weight(hd + 6, hd)
    kw = C.norm_weight(hd + 7, hd)
    ct, st = oracle.rope_tables(T + 3, hd, 1e6)
    pos = (np.arange(T) + 3).astype(np.int32)
    q_np = qkv[:, :Hq * hd].reshape(T, Hq, hd)
    k_np = qkv[:, Hq * hd:(Hq + Hk) * hd].reshape(T, Hk, hd)
    want_q = oracle.rmsnorm_rope(q_np, qw, ct, st, pos, 1e-6)
    want_k = oracle.rmsnorm_rope(k_np, kw, ct, st, pos, 1e-6)
    t = dev(qkv)
    q = t[:, :Hq * hd].view(T, Hq, hd)
    k = t[:, Hq * hd:(Hq + Hk) * hd].view(T, Hk, hd)
    cache = torch.zeros((T + 4, Hk, hd), dtype=torch.float16, device="cuda")
    ops.qk_rmsnorm_rope(q, k, dev(qw), dev(kw), dev(ct), dev(st), positions=dev(pos), eps=1e-6,
                        k_cache=cache[2:2 + T], keep_k_f32=keep)
    out = host(t)
    assert_bits(out[:, :Hq * hd].reshape(T, Hq, hd), want_q, "q")
    assert_bits(out[:, Hq * hd:(Hq + Hk) * hd].reshape(T, Hk, hd), want_k if keep else k_np, "k f32")
    c = host(cache).view(np.uint16)
    assert_bits(c[2:2 + T], oracle.kv_pack_f16(want_k), "k cache")
    assert not c[:2].any() and not c[2 + T:].any()


# --------------------------------------------------------------------------- RoPE only, the fused Q/K/V stage

@pytest.mark.parametrize("H", [3, 8])
@pytest.mark.parametrize("hd", [64, 96, 128, 256])
def test_rope_only_heads_tokens(ops, oracle, hd, H):
    T = 41
    buf = C.normal(hd + 40, (T, H, hd))
    ct, st = oracle.rope_tables(64, hd, 1e4)
    pos = C.rng(hd).integers(0, 64, T).astype(np.int32)
    pos[0] = 0
    bt = dev(buf)
    ops.rope_only_heads(bt, dev(ct), dev(st), positions=dev(pos))
    assert_bits(host(bt), oracle.rope_only(buf, ct, st, pos), f"rope only hd={hd} H={H}")


@pytest.mark.parametrize("heads", [(6, 2), (16, 8)])
@pytest.mark.parametrize("norm", [True, False])
@pytest.mark.parametrize("bias", [True, False])
@pytest.mark.parametrize("hd", [128, 96])
def test_qkv_stage_matches_the_per_token_calls(ops, oracle, norm, bias, hd, heads):
    """One launch == Stage C of the Q8 prefill per token (src/asm/prefill_q8.inc:848-883): bias add, Q/K
    RMSNorm+RoPE (Qwen3) or RoPE only (Llama), K and V binary16 cache rows.  16 + 8 + 8 heads of 128 run
    the wave-uniform kernel."""
    T = 53
    Hq, Hk = heads
    w = (Hq + 2 * Hk) * hd
    qkv = C.normal(hd + 90, (T, w))
    qw, kw = C.norm_weight(hd + 91, hd), C.norm_weight(hd + 92, hd)
    qb = C.normal(hd + 93, Hq * hd, 0.5) if bias else None
    kb = C.normal(hd + 94, Hk * hd, 0.5) if bias else None
    vb = C.normal(hd + 95, Hk * hd, 0.5) if bias else None
    ct, st = oracle.rope_tables(T + 10, hd, 1e6)
    pos = (np.arange(T) + 10).astype(np.int32)
    pos[3] = 0
    q_np = qkv[:, :Hq * hd].reshape(T, Hq, hd)
    k_np = qkv[:, Hq * hd:(Hq + Hk) * hd].reshape(T, Hk, hd)
    v_np = qkv[:, (Hq + Hk) * hd:].reshape(T, Hk, hd)
    wq, wk, wv, wkc, wvc = oracle.qkv_stage(q_np, k_np, v_np, qw if norm else None, kw if norm else None, qb, kb, vb,
                                            ct, st, pos, 1e-6)
    t = dev(qkv)
    q = t[:, :Hq * hd].view(T, Hq, hd)
    k = t[:, Hq * hd:(Hq + Hk) * hd].view(T, Hk, hd)
    v = t[:, (Hq + Hk) * hd:].view(T, Hk, hd)
    kc = torch.zeros((T, Hk, hd), dtype=torch.float16, device="cuda")
    vc = torch.zeros((T, Hk, hd), dtype=torch.float16, device="cuda")
    d = lambda a: None if a is None else dev(a)  # noqa: E731
    ops.qkv_rope_stage(q, k, v, dev(ct), dev(st), positions=dev(pos), eps=1e-6,
                       q_norm_weight=d(qw) if norm else None, k_norm_weight=d(kw) if norm else None,
                       q_bias=d(qb), k_bias=d(kb), v_bias=d(vb), k_cache=kc, v_cache=vc)
    out = host(t)
    assert_bits(out[:, :Hq * hd].reshape(T, Hq, hd), wq, "q")
    assert_bits(out[:, Hq * hd:(Hq + Hk) * hd].reshape(T, Hk, hd), wk, "k")
    assert_bits(out[:, (Hq + Hk) * hd:].reshape(T, Hk, hd), wv, "v")
    assert_bits(host(kc).view(np.uint16), wkc, "k cache")
    assert_bits(host(vc).view(np.uint16), wvc, "v cache")


@pytest.mark.parametrize("heads", [(4, 2), (8, 8)])
def test_qkv_stage_cache_only_leaves_f32_k_v(ops, oracle, heads):
    T, hd = 9, 128
    Hq, Hk = heads
    qkv = C.normal(7, (T, (Hq + 2 * Hk) * hd))
    ct, st = oracle.rope_tables(T, hd, 1e6)
    pos = np.arange(T, dtype=np.int32)
    q_np = qkv[:, :Hq * hd].reshape(T, Hq, hd)
    k_np = qkv[:, Hq * hd:(Hq + Hk) * hd].reshape(T, Hk, hd)
    v_np = qkv[:, (Hq + Hk) * hd:].reshape(T, Hk, hd)
    qw, kw = C.norm_weight(8, hd), C.norm_weight(9, hd)
    wq, wk, wv, wkc, wvc = oracle.qkv_stage(q_np, k_np, v_np, qw, kw, None, None, None, ct, st, pos, 1e-6)
    t = dev(qkv)
    kc = torch.zeros((T, Hk, hd), dtype=torch.float16, device="cuda")
    vc = torch.zeros((T, Hk, hd), dtype=torch.float16, device="cuda")
    ops.qkv_rope_stage(t[:, :Hq * hd].view(T, Hq, hd), t[:, Hq * hd:(Hq + Hk) * hd].view(T, Hk, hd),
                       t[:, (Hq + Hk) * hd:].view(T, Hk, hd), dev(ct), dev(st), positions=dev(pos),
                       q_norm_weight=dev(qw), k_norm_weight=dev(kw), k_cache=kc, v_cache=vc, keep_k_f32=False,
                       keep_v_f32=False)
    out = host(t)
    assert_bits(out[:, :Hq * hd].reshape(T, Hq, hd), wq, "q")
    assert_bits(out[:, Hq * hd:], qkv[:, Hq * hd:], "k and v f32 untouched")
    assert_bits(host(kc).view(np.uint16), wkc, "k cache")
    assert_bits(host(vc).view(np.uint16), wvc, "v cache")


def test_ops_bind_to_torchs_current_stream(ops):
    """The torch-facing entries launch on torch's current stream: the raw stream query they use agrees with
    torch.cuda.current_stream() on the default stream, inside a stream context and under graph capture, where
    a captured call runs only when the graph replays."""
    from v7multiplikator_amd import _lib
    dev = torch.device("cuda", torch.cuda.current_device())
    assert ops.current_stream_handle(dev) == torch.cuda.current_stream().cuda_stream
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        assert ops.current_stream_handle(dev) == side.cuda_stream
        x = torch.zeros(4096, device="cuda")
        ops.add_inplace(x, torch.ones(4096, device="cuda"))
    side.synchronize()
    assert bool((x == 1).all())
    x = torch.zeros(4096, device="cuda")
    y = torch.full((4096,), 2.0, device="cuda")
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    seen = []
    try:
        with torch.cuda.graph(g):
            seen.append((ops.current_stream_handle(dev), torch.cuda.current_stream().cuda_stream))
            ops.add_inplace(x, y)
    finally:
        _lib.load().v7g_set_stream(torch.cuda.current_stream().cuda_stream)
    assert seen[0][0] == seen[0][1]
    torch.cuda.synchronize()
    assert bool((x == 0).all())  # captured, not run
    g.replay()
    g.replay()
    torch.cuda.synchronize()
    assert bool((x == 4).all())


def test_time_next_call_binds_kernel_timestamps(ops):
    """v7g_time_next_call: the armed events time exactly the next launching call, from its kernels'
    own timestamps; a rejected call keeps the pair armed; later calls leave the events alone."""
    from v7multiplikator_amd import _lib
    L = _lib.load()
    torch.cuda.synchronize()
    L.v7g_set_stream(torch.cuda.current_stream().cuda_stream)
    stream = torch.cuda.current_stream()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(stream)
    b.record(stream)
    rows, hidden = 2048, 8192
    g = torch.randn(rows, hidden, device="cuda")
    u = torch.randn(rows, hidden, device="cuda")
    q = torch.empty(rows, hidden, dtype=torch.int8, device="cuda")
    s = torch.empty(rows, hidden // 32, device="cuda")
    assert L.v7g_time_next_call(a.cuda_event, b.cuda_event) == 0
    # rejected (group size 0): launches nothing, the pair stays armed
    assert L.v7g_swiglu_q8(q.data_ptr(), s.data_ptr(), g.data_ptr(), u.data_ptr(), rows, hidden, 0) != 0
    L.v7g_clear_last_error()
    assert L.v7g_swiglu_q8(q.data_ptr(), s.data_ptr(), g.data_ptr(), u.data_ptr(), rows, hidden, 32) == 0
    torch.cuda.synchronize()
    ms = a.elapsed_time(b)
    # 2048 x 8192 SwiGLU -> Q8 moves 153 MB: between 15 us (10 TB/s) and 10 ms
    assert 0.015 < ms < 10.0, ms
    # the pair is disarmed: a further call does not move the events
    assert L.v7g_swiglu_q8(q.data_ptr(), s.data_ptr(), g.data_ptr(), u.data_ptr(), rows, hidden, 32) == 0
    torch.cuda.synchronize()
    assert a.elapsed_time(b) == ms
    assert L.v7g_get_last_error() == 0


def test_host_threads_drive_their_own_streams(ops, oracle):
    """Two host threads, each on its own stream (the library binds the stream per thread), run SwiGLU->Q8 and
    add+RMSNorm concurrently; every result equals the oracle bit for bit."""
    import threading

    g = C.normal(7001, (64, 4096), 1.5)
    u = C.normal(7002, (64, 4096), 1.5)
    res = C.normal(7003, (64, 4096))
    add = C.normal(7004, (64, 4096))
    w = C.norm_weight(7005, 4096)
    want_q, want_s = oracle.swiglu_q8(g, u, 32)
    want_o, want_r = oracle.fused_add_rmsnorm(res, add, w, 1e-6)
    errors = []

    def worker(kind):
        try:
            stream = torch.cuda.Stream()
            with torch.cuda.stream(stream):
                for _ in range(20):
                    if kind == "q8":
                        q, s = ops.swiglu_q8(dev(g), dev(u), gs=32)
                        stream.synchronize()
                        assert np.array_equal(q.cpu().numpy(), want_q) and np.array_equal(s.cpu().numpy(), want_s)
                    else:
                        r = dev(res)
                        o = ops.fused_add_rmsnorm(r, dev(add), dev(w), eps=1e-6)
                        stream.synchronize()
                        assert np.array_equal(o.cpu().numpy(), want_o) and np.array_equal(r.cpu().numpy(), want_r)
        except BaseException as e:  # noqa: BLE001 -- reported by the main thread
            errors.append((kind, repr(e)))

    threads = [threading.Thread(target=worker, args=(k,)) for k in ("q8", "norm")]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=60)
    assert not any(t.is_alive() for t in threads)
    assert not errors, errors


def test_chain_captured_in_a_hip_graph(ops, oracle):
    """The four chain kernels captured in one HIP graph (torch.cuda.graph) and replayed three times, with eager
    work between the replays: every replay equals the eager run bit for bit.  The kernels use no memset nodes
    and allocate nothing, so they are safe to capture."""
    T, D, V, NQ, NKV, HD, HID = 64, 512, 1000, 4, 2, 128, 1024
    tq, ts = C.q8_table(8101, V, D)
    ids = dev(C.rng(8102).integers(0, V, T).astype(np.int32))
    res0 = dev(C.normal(8103, (T, D)))
    add = dev(C.normal(8104, (T, D)))
    w = dev(C.norm_weight(8105, D))
    qkv0 = dev(C.normal(8106, (T, (NQ + 2 * NKV) * HD)))
    qw, kw = dev(C.norm_weight(8107, HD)), dev(C.norm_weight(8108, HD))
    ct, st = (dev(a) for a in oracle.rope_tables(T, HD, 1e6))
    pos = dev(np.arange(T, dtype=np.int32))
    gate, up = dev(C.normal(8109, (T, HID), 1.5)), dev(C.normal(8110, (T, HID), 1.5))
    tqd, tsd = dev(tq), dev(ts)
    emb = torch.empty((T, D), device="cuda")
    normed = torch.empty((T, D), device="cuda")
    codes = torch.empty((T, HID), dtype=torch.int8, device="cuda")
    scales = torch.empty((T, HID // 32), device="cuda")
    res, qkv = res0.clone(), qkv0.clone()

    def chain():
        ops.embedding_gather_q8(ids, tqd, tsd, out=emb)
        ops.fused_add_rmsnorm(res, add, w, eps=1e-6, out=normed)
        q = qkv[:, :NQ * HD].view(T, NQ, HD)
        k = qkv[:, NQ * HD:(NQ + NKV) * HD].view(T, NKV, HD)
        ops.qk_rmsnorm_rope(q, k, qw, kw, ct, st, positions=pos, eps=1e-6)
        ops.swiglu_q8(gate, up, gs=32, out_q=codes, out_s=scales)

    def snapshot():
        torch.cuda.synchronize()
        return [t.cpu().numpy().copy() for t in (emb, res, normed, qkv, codes, scales)]

    chain()
    want = snapshot()
    res.copy_(res0)
    qkv.copy_(qkv0)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        chain()  # warm-up on the capture stream, as torch recommends
    torch.cuda.current_stream().wait_stream(side)
    with torch.cuda.graph(g):
        chain()
    for replay in range(3):
        for t in (emb, normed, codes, scales):
            t.zero_()
        res.copy_(res0)
        qkv.copy_(qkv0)
        torch.cuda.synchronize()
        g.replay()
        got = snapshot()
        for name, a, b in zip(("emb", "residual", "normed", "qkv", "codes", "scales"), got, want):
            assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), (replay, name)


def test_rope_tables_llama3_match_oracle(ops, oracle):
    """Llama 3 scaled tables built by the library (host, extended precision) equal the oracle's bit for bit,
    through the caller-owned builder and the library-owned v7g_rope_init_llama3; a RMSNorm+RoPE pass over them
    is bit-exact too."""
    import ctypes

    from v7multiplikator_amd import _lib
    p = dict(factor=8.0, low_freq_factor=1.0, high_freq_factor=4.0, original_max_position_embeddings=8192)
    P, D, base = 4096, 128, 500000.0
    wc, ws = oracle.rope_tables_llama3(P, D, base, 8.0, 1.0, 4.0, 8192)
    c, s = ops.rope_tables(P, D, base, llama3=p)
    assert_bits(host(c), wc, "cos")
    assert_bits(host(s), ws, "sin")
    L = _lib.load()
    assert L.v7g_rope_init_llama3(D, ctypes.c_float(base), P, ctypes.c_float(8.0), ctypes.c_float(1.0),
                                  ctypes.c_float(4.0), 8192) == 0
    cp, sp, rmd, npos = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_int(), ctypes.c_int()
    assert L.v7g_get_rope_tables(ctypes.byref(cp), ctypes.byref(sp), ctypes.byref(rmd), ctypes.byref(npos)) == 0
    assert rmd.value == D // 2 and npos.value == P
    tc = torch.empty((P, D // 2), device="cuda")
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    assert hip.hipMemcpy(tc.data_ptr(), cp.value, tc.numel() * 4, 3) == 0  # hipMemcpyDeviceToDevice
    assert_bits(host(tc), wc, "owned cos")
    T, H = 64, 8
    buf = C.normal(8201, (T, H, D))
    w = C.norm_weight(8202, D)
    pos = C.rng(8203).integers(0, P, T).astype(np.int32)
    bt = dev(buf)
    ops.rmsnorm_rope_heads(bt, dev(w), c, s, positions=dev(pos), eps=1e-6)
    assert_bits(host(bt), oracle.rmsnorm_rope(buf, w, wc, ws, pos, 1e-6), "rope over llama3 tables")
    # restore the plain library-owned tables the drop-in test expects to be replaceable
    assert L.v7g_rope_init(D, ctypes.c_float(1e6), 16) == 0


def test_pointer_checks_reject_host_memory(ops):
    """With pointer checks on, a pageable host buffer is rejected with V7G_ERR_ADDRESS before any launch, while
    device memory and pinned host memory pass; with checks off (the default) nothing is queried."""
    from v7multiplikator_amd import _lib
    L = _lib.load()
    n = 4096
    host_x = np.ones(n, np.float32)  # pageable host memory: the GPU must never see this pointer
    dx = torch.ones(n, device="cuda")
    dy = torch.ones(n, device="cuda")
    pinned = torch.ones(n, dtype=torch.float32).pin_memory()
    L.v7g_set_stream(torch.cuda.current_stream().cuda_stream)
    # classify first, launching nothing: the entry below is only called with the host pointer once the
    # runtime is known to report it as inaccessible
    assert L.v7g_check_pointer(host_x.ctypes.data) == _lib.V7G_ERR_ADDRESS
    assert L.v7g_check_pointer(dx.data_ptr()) == 0 and L.v7g_check_pointer(pinned.data_ptr()) == 0
    try:
        L.v7g_set_pointer_checks(1)
        L.v7g_clear_last_error()
        assert L.v7g_add_inplace(host_x.ctypes.data, dy.data_ptr(), n) == _lib.V7G_ERR_ADDRESS
        assert L.v7g_get_last_error() == _lib.V7G_ERR_ADDRESS
        L.v7g_clear_last_error()
        assert L.v7g_add_inplace(dx.data_ptr(), dy.data_ptr(), n) == 0
        assert L.v7g_add_inplace(dx.data_ptr(), pinned.data_ptr(), n) == 0
        torch.cuda.synchronize()
        assert torch.all(dx == 3.0).item()
        assert L.v7g_get_last_error() == 0
    finally:
        L.v7g_set_pointer_checks(0)
        L.v7g_clear_last_error()


def test_torch_ops_reject_undersized_outputs_and_mismatched_tables(ops):
    """The torch-facing functions refuse, before any launch, buffers the kernels would overrun: outputs of
    another shape, norm weights that are not [head_dim], cos/sin tables of different shapes."""
    r = torch.zeros((4, 256), device="cuda")
    a = torch.zeros((4, 256), device="cuda")
    w = torch.ones(256, device="cuda")
    with pytest.raises(ValueError):
        ops.fused_add_rmsnorm(r, a, w, out=torch.empty((2, 256), device="cuda"))
    with pytest.raises(ValueError):
        ops.swiglu(r, a, out=torch.empty(100, device="cuda"))
    ids = torch.zeros(3, dtype=torch.int32, device="cuda")
    tq = torch.zeros((10, 128), dtype=torch.int8, device="cuda")
    ts = torch.ones(10 * 2, device="cuda")
    with pytest.raises(ValueError):
        ops.embedding_gather_q8(ids, tq, ts, out=torch.empty((2, 128), device="cuda"))
    q = torch.zeros((2, 4, 128), device="cuda")
    k = torch.zeros((2, 2, 128), device="cuda")
    qw = torch.ones(128, device="cuda")
    c = torch.ones((4, 64), device="cuda")
    with pytest.raises(ValueError):
        ops.rmsnorm_rope_heads(q, torch.ones(64, device="cuda"), c, c)
    with pytest.raises(ValueError):
        ops.rmsnorm_rope_heads(q, qw, c, torch.ones((2, 64), device="cuda"))
    with pytest.raises(ValueError):
        ops.qk_rmsnorm_rope(q, k, qw, torch.ones(96, device="cuda"), c, c)
    with pytest.raises(ValueError):
        ops.rope_only_heads(q, c, torch.ones((4, 32), device="cuda"))
    with pytest.raises(ValueError):
        ops.qkv_rope_stage(q, k, None, c, c, q_norm_weight=torch.ones(64, device="cuda"))
    torch.cuda.synchronize()
    # the valid calls still run
    ops.rmsnorm_rope_heads(q, qw, c, c)
    ops.fused_add_rmsnorm(r, a, w)
    torch.cuda.synchronize()


# --------------------------------------------------------------------------- denormal data: the reference's FTZ + DAZ

F = np.float32


def denormal_mix(seed, shape):
    """Rows of four kinds, cycled: denormals (random bits), tiny normals whose squares and products are
    denormal (N(0,1) * 2^-66), values just above 2^-126, and ordinary N(0,1) values sprinkled with all three."""
    rng = C.rng(seed)
    rows = int(np.prod(shape[:-1]))
    n = shape[-1]
    x = np.empty((rows, n), F)
    for r in range(rows):
        kind = r % 4
        if kind == 0:
            bits = rng.integers(0, 0x00800000, n, dtype=np.uint32) | (rng.integers(0, 2, n, dtype=np.uint32) << 31)
            x[r] = bits.view(F)
        elif kind == 1:
            x[r] = rng.standard_normal(n).astype(F) * F(2.0 ** -66)
        elif kind == 2:
            x[r] = (F(2.0 ** -126) * (1 + rng.random(n))).astype(F) * rng.choice(np.array([-1, 1], F), n)
        else:
            x[r] = rng.standard_normal(n).astype(F)
            pick = rng.integers(0, n, n // 4)
            x[r, pick] = (rng.standard_normal(pick.size) * 2.0 ** -128).astype(F)
    return x.reshape(shape)


@pytest.mark.parametrize("eps", [0.0, 1e-6])
@pytest.mark.parametrize("dim", [256, 4096])
def test_denormal_rows_norms_follow_ftz_daz(ops, oracle, eps, dim):
    """add+RMSNorm, RMSNorm, RMSNorm->Q8 and the fused add->RMSNorm->Q8 on rows of denormals and tiny values,
    bit for bit with the oracle in the reference's MXCSR FTZ+DAZ mode (eps = 0 lets an all-flushed sum of
    squares give an infinite scale).  dim 4096 takes the 16-elements-per-thread RMSNorm->Q8 kernel."""
    r = denormal_mix(501, (16, dim))
    a = denormal_mix(502, (16, dim))[::-1].copy()
    w = C.norm_weight(503, dim)
    wo, wr = oracle.fused_add_rmsnorm(r, a, w, eps)
    rt = dev(r)
    o = ops.fused_add_rmsnorm(rt, dev(a), dev(w), eps=eps)
    assert_bits(host(rt), wr, "residual")
    assert_bits(host(o), wo, "o")
    assert_bits(host(ops.rmsnorm(dev(r), dev(w), eps=eps)), oracle.rmsnorm(r, w, eps), "rmsnorm")
    for gs in (32, 64):
        q, sc = ops.rmsnorm_quantize(dev(r), dev(w), eps=eps, gs=gs)
        wq, ws = oracle.rmsnorm_quantize(r, w, eps, gs)
        assert_bits(host(q), wq, "codes")
        assert_bits(host(sc), ws, "scales")
        q, sc = ops.add_rmsnorm_quantize(dev(r), dev(a), dev(w), eps=eps, gs=gs)
        wq, ws = oracle.rmsnorm_quantize(oracle.add_inplace(r, a), w, eps, gs)
        assert_bits(host(q), wq, "fused codes")
        assert_bits(host(sc), ws, "fused scales")


def test_denormal_heads_rope_follow_ftz_daz(ops, oracle):
    """Q/K RMSNorm+RoPE, RoPE only and the Q/K/V stage with bias on heads of denormals and tiny values."""
    T, HQ, HK, D = 8, 8, 4, 128
    q = denormal_mix(511, (T, HQ, D))
    k = denormal_mix(512, (T, HK, D))
    qw = C.norm_weight(513, D)
    kw = C.norm_weight(514, D)
    ct, st = oracle.rope_tables(T, D, 1e6)
    pos = np.arange(T, dtype=np.int32)
    qt, kt = dev(q), dev(k)
    ops.qk_rmsnorm_rope(qt, kt, dev(qw), dev(kw), dev(ct), dev(st), positions=dev(pos), eps=1e-6)
    assert_bits(host(qt), oracle.rmsnorm_rope(q, qw, ct, st, pos, 1e-6), "q")
    assert_bits(host(kt), oracle.rmsnorm_rope(k, kw, ct, st, pos, 1e-6), "k")
    bt = dev(q)
    ops.rope_only_heads(bt, dev(ct), dev(st), positions=dev(pos))
    assert_bits(host(bt), oracle.rope_only(q, ct, st, pos), "rope only")
    v = denormal_mix(515, (T, HK, D))
    qb = denormal_mix(516, (HQ * D,))
    kb = denormal_mix(517, (HK * D,))
    vb = denormal_mix(518, (HK * D,))
    want = oracle.qkv_stage(q, k, v, qw, kw, qb, kb, vb, ct, st, pos, 1e-6)
    qt, kt, vt = dev(q), dev(k), dev(v)
    kc = torch.empty((T, HK, D), dtype=torch.float16, device="cuda")
    vc = torch.empty((T, HK, D), dtype=torch.float16, device="cuda")
    ops.qkv_rope_stage(qt, kt, vt, dev(ct), dev(st), positions=dev(pos), eps=1e-6, q_norm_weight=dev(qw),
                       k_norm_weight=dev(kw), q_bias=dev(qb), k_bias=dev(kb), v_bias=dev(vb), k_cache=kc, v_cache=vc)
    for got, exp, name in zip((host(qt), host(kt), host(vt)), want[:3], ("q", "k", "v")):
        assert_bits(got, exp, f"stage {name}")
    assert_bits(host(kc).view(np.uint16), oracle.kv_pack_f16(want[1].reshape(T, -1)).reshape(T, HK, D), "k cache")
    assert_bits(host(vc).view(np.uint16), oracle.kv_pack_f16(want[2].reshape(T, -1)).reshape(T, HK, D), "v cache")


@pytest.mark.parametrize("rows,row_len", [(32, 4096), (12, 1000)])
def test_denormal_swiglu_and_quantize_follow_ftz_daz(ops, oracle, rows, row_len):
    """SwiGLU, SwiGLU->Q8, Q8 quantize (flat and general paths), add and the binary16 pack on denormal data;
    quantizer groups whose max is below 2^-118 are where a denormal element's code depends on DAZ."""
    g = denormal_mix(521, (rows, row_len))
    u = denormal_mix(522, (rows, row_len))[::-1].copy()
    assert_bits(host(ops.swiglu(dev(g), dev(u))), oracle.swiglu(g, u), "swiglu")
    x = g.copy()
    x[1::4] = (x[1::4] * F(2.0 ** -54)).astype(F)  # group maxima near 2^-120: the floor scale meets denormals
    for gs in (32, 64):
        wq, ws = oracle.swiglu_q8(g, u, gs)
        gq, gsc = ops.swiglu_q8(dev(g), dev(u), gs=gs)
        assert_bits(host(gq), wq, "swiglu_q8 codes")
        assert_bits(host(gsc), ws, "swiglu_q8 scales")
        wq, ws = oracle.quantize(x, gs)
        gq, gsc = ops.quantize_q8(dev(x), gs=gs)
        assert_bits(host(gq), wq, "quantize codes")
        assert_bits(host(gsc), ws, "quantize scales")
    assert_bits(host(ops.add_inplace(dev(g), dev(u))), oracle.add_inplace(g, u), "add_inplace")
    if row_len % 4 == 0:
        assert_bits(host(ops.kv_pack_f16(dev(g))).view(np.uint16), oracle.kv_pack_f16(g), "kv pack")
