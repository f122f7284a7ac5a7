"""Pins of the CPU oracle (oracle/v7_oracle.c, oracle/oracle.py) -- CPU only.

The oracle restates the reference NASM kernels operation by operation.  These
tests pin it with facts that do not come from the oracle itself:

  * hand-derived known answers that only the reference's accumulation order
    produces (sum of squares: four 8-lane accumulators, leftover blocks first
    into A, (A+B)+(C+D), HADD_YMM; src/asm/add_rmsnorm_kernel.inc:29-73,
    src/asm/v7_macros.inc:38-45,263-291);
  * the reference validators' own checks: kt_quantize_c_ref exact codes on
    the seven KTPAT patterns (tools/kt_utils.h:139-191,378-407,681-731), the
    double-precision RMSNorm+RoPE reference and float add+RMSNorm reference
    within 1e-3 (tools/kt_utils.h:450-503,820,935-1074);
  * closed forms and invariants: exact int8 x f32 dequant, the quantizer's
    all-zero-group scale 2^-126, absmax -> +-127, rotations by 0 and 90
    degrees, pos = 0 without rotation, pair norms, sigmoid/SwiGLU against
    double precision;
  * the AVX2 restatement (the CPU baseline) against the scalar oracle, bit for bit.
"""
from __future__ import annotations

import ctypes
import math

import numpy as np
import pytest

from tests import common as C

F = np.float32
TWO24 = float(2 ** 24)


def bits_equal(a, b):
    a = np.asarray(a)
    b = np.asarray(b)
    if a.shape != b.shape:
        return False
    if a.dtype.kind == "f":
        return bool(np.array_equal(a.view(np.uint32 if a.dtype == np.float32 else np.uint64),
                                   b.view(np.uint32 if b.dtype == np.float32 else np.uint64)))
    return bool(np.array_equal(a, b))


# --------------------------------------------------------------------------- sum of squares order (a1, a2, a3)

def test_sumsq_hadd_tree_known_answer(oracle):
    """dim 32: x[0] = 4096 (square 2^24), x[1..7] = 1, rest 0.  Only accumulator A is non-zero, so the
    HADD_YMM input is v = [2^24, 1, 1, 1, 1, 1, 1, 1]:
      s0 = v0 + v4 = 2^24 + 1 -> 2^24 (tie to even), s1 = s2 = s3 = 2,
      (s0 + s1) + (s2 + s3) = (2^24 + 2) + 4 = 2^24 + 6.
    A left-to-right sum gives 2^24 (every +1 is absorbed)."""
    x = np.zeros(32, F)
    x[0] = 4096.0
    x[1:8] = 1.0
    assert float(oracle.sumsq_lanes(x)) == TWO24 + 6


def test_sumsq_accumulator_interleave_known_answer(oracle):
    """dim 64 (8 blocks, 2 groups): blocks 0,4 -> A, 1,5 -> B, 2 -> C, 3 -> D, lane 0 only.
    x[0] = 4096 (A), x[32] = 1 (A: fma(1,1,2^24) = 2^24), x[8] = x[40] = 1 (B = 2), x[16] = 1 (C), x[24] = 1 (D):
      v0 = (A + B) + (C + D) = (2^24 + 2) + 2 = 2^24 + 4.
    One accumulator per lane in element order gives 2^24."""
    x = np.zeros(64, F)
    x[0] = 4096.0
    for i in (8, 16, 24, 32, 40):
        x[i] = 1.0
    assert float(oracle.sumsq_lanes(x)) == TWO24 + 4


def test_sumsq_leftover_blocks_first_known_answer(oracle):
    """dim 40 (5 blocks, 1 leftover): the leftover block 0 goes first into A, then blocks 1..4 feed A, B, C, D.
    x[0] = 4096 (block 0 -> A), x[24] = 1 (block 3 -> C), x[32] = 1 (block 4 -> D):
      v0 = (2^24 + 0) + (1 + 1) = 2^24 + 2.
    Were the leftover block taken last (blocks 0..3 -> A..D, block 4 -> A), block 4 would be absorbed into A
    and block 3 would land in D: (2^24 + 0) + (0 + 1) = 2^24 (tie to even)."""
    x = np.zeros(40, F)
    x[0] = 4096.0
    x[24] = 1.0
    x[32] = 1.0
    assert float(oracle.sumsq_lanes(x)) == TWO24 + 2


def test_sumsq_hadd_pairing_known_answer(oracle):
    """dim 32 with only block 0 non-zero, so the HADD_YMM input is v = x[0:8]^2 = [0, 9, 0, 2^24, 16, 9, 1, 9]:
      s0 = v0 + v4 = 16, s1 = v1 + v5 = 18, s2 = v2 + v6 = 1, s3 = v3 + v7 = 2^24 + 9 -> 2^24 + 8 (tie to even),
      t0 = s0 + s1 = 34, t2 = s2 + s3 = 2^24 + 9 -> 2^24 + 8, t0 + t2 = 2^24 + 42.
    Pairing adjacent lanes, summing left to right, (s0 + s2) + (s1 + s3) or a sequential sum all give
    2^24 + 40, 2^24 + 44 or similar instead."""
    x = np.zeros(32, F)
    x[:8] = [0, 3, 0, 4096, 4, 3, 1, 3]
    assert float(oracle.sumsq_lanes(x)) == TWO24 + 42


def test_sumsq_chains_are_fused_known_answer(oracle):
    """dim 64: lane 0 of accumulator A takes x[0] = 2 then x[32] = 1 + 2^-23 (blocks 0 and 4).  With FMA the
    chain is RN(4 + (1 + 2^-22 + 2^-46)) = 5 + 2^-21 (more than half an ulp above 5); a separate multiply
    drops the 2^-46 first and the tie 5 + 2^-22 rounds to 5."""
    x = np.zeros(64, F)
    x[0] = 2.0
    x[32] = F(1.0) + F(2.0 ** -23)
    assert float(oracle.sumsq_lanes(x)) == 5.0 + 2.0 ** -21


def test_rms_scale_step_roundings_known_answers(oracle):
    """COMPUTE_RMS_SCALE rounds after each of vdivss, vaddss, vsqrtss, vdivss:
      * sumsq/dim by division: sumsq = 24 + 2^-18, dim 24: 1 + 2^-23 (times RN(1/24) would give 1 + 2^-22),
        whose square root lies below the midpoint 1 + 2^-24 and rounds to 1, so the scale is exactly 1
        (1 + 2^-22 would give 1 - 2^-23);
      * 1/sqrt in two roundings: mean v = 1.0000044107437134 gives RN(1/RN(sqrt v)) = 0.9999978542327881,
        where the correctly rounded 1/sqrt(v) is 0.9999977946281433."""
    assert float(oracle.rms_scale(F(24.0) + F(2.0 ** -18), 24, 0.0)) == 1.0
    v = F(1.0000044107437134)
    assert float(oracle.rms_scale(F(v * F(64)), 64, 0.0)) == float(F(0.9999978542327881))


def test_rms_scale_closed_form(oracle):
    """COMPUTE_RMS_SCALE = 1/sqrt(sumsq/n + eps) in four correctly rounded steps: exact for powers of two."""
    assert float(oracle.rms_scale(F(4 * 64), 64, 0.0)) == 0.5
    assert float(oracle.rms_scale(F(64), 64, 0.0)) == 1.0
    # each step rounded to binary32 (numpy float32 ops are IEEE binary32)
    ss, n, eps = F(123.456), 128, F(1e-6)
    want = F(1.0) / np.sqrt(F(ss / F(n)) + eps)
    assert bits_equal(np.array([oracle.rms_scale(ss, n, float(eps))], F), np.array([want], F))


def test_fused_add_rmsnorm_constant_row_closed_form(oracle):
    """x = residual + add = 2 everywhere, w = 1, eps = 0: sumsq = 4*dim exactly, scale = 1/2, o = 1 exactly."""
    for dim in (8, 24, 64, 4096):
        r = np.full((1, dim), 1.5, F)
        a = np.full((1, dim), 0.5, F)
        o, rr = oracle.fused_add_rmsnorm(r, a, np.ones(dim, F), 0.0)
        assert np.all(rr == 2.0) and np.all(o == 1.0)


@pytest.mark.parametrize("dim", [8, 16, 24, 48, 64, 128, 256, 1024, 2048, 3072, 4096, 8192])
@pytest.mark.parametrize("seed", [12345, 67890])
def test_fused_add_rmsnorm_vs_validator_refs(oracle, dim, seed):
    """tools/v_rmsnorm_validate.cpp:87-101 shapes: within 1e-3 of the float C reference (the reference's own
    tolerance, tools/kt_utils.h:820) and within 1e-5 relative of a double-precision evaluation."""
    r = C.validator_row(seed, dim)
    a = C.validator_row(seed + 1, dim)
    w = C.validator_weight(seed + 2, dim)
    o, rr = oracle.fused_add_rmsnorm(r[None], a[None], w, 1e-6)
    assert bits_equal(rr[0], (r + a).astype(F))  # residual update: one binary32 add per element
    ko, _ = oracle.kt_fused_add_rmsnorm_c_ref(r, a, w, 1e-6)
    assert np.max(np.abs(o[0] - ko)) < 1e-3
    x = (r + a).astype(np.float64)
    d = x / np.sqrt(np.mean(x * x) + 1e-6) * w.astype(np.float64)
    assert np.max(np.abs(o[0] - d) / np.maximum(np.abs(d), 1e-3)) < 1e-5


def test_fused_add_rmsnorm_benchmark_distribution(oracle):
    """[64, 2048] ~N(0,1), w = 1+N(0,0.1): max relative error vs double below 1e-5 (the f32 bar)."""
    r = C.normal(101, (64, 2048))
    a = C.normal(102, (64, 2048))
    w = C.norm_weight(103, 2048)
    o, _ = oracle.fused_add_rmsnorm(r, a, w, 1e-6)
    x = r.astype(np.float64) + a.astype(np.float64)
    x = x.astype(F).astype(np.float64)
    d = x / np.sqrt(np.mean(x * x, axis=1, keepdims=True) + 1e-6) * w
    rel = np.abs(o - d) / np.abs(d)
    assert np.max(rel[np.abs(d) > 1e-6]) < 1e-5


# --------------------------------------------------------------------------- RMSNorm + RoPE (a3, a4)

def _normed(oracle, x, w, eps):
    """pos-0 output: (x*scale)*w with the lane-ordered scale; used to state the rotation invariants."""
    return oracle.rmsnorm_rope(x, w, np.ones((1, x.shape[-1] // 2), F), np.zeros((1, x.shape[-1] // 2), F),
                               np.zeros(x.shape[0], np.int32), eps)


def test_rope_pos0_is_rmsnorm_only(oracle):
    x = C.normal(1, (3, 4, 128))
    w = C.norm_weight(2, 128)
    ct, st = oracle.rope_tables(4, 128, 1e6)
    got = oracle.rmsnorm_rope(x, w, ct, st, np.zeros(3, np.int32), 1e-6)
    s = np.array([[oracle.rms_scale(oracle.sumsq_lanes(x[t, h]), 128, 1e-6) for h in range(4)] for t in range(3)], F)
    want = ((x * s[..., None]).astype(F) * w).astype(F)
    assert bits_equal(got, want)


def test_rope_quarter_turn_and_identity_tables(oracle):
    """cos = 0, sin = 1 at pos 1: out_j = -xo, out_{j+h} = xe exactly (fma(-xo, 1, xe*0), fma(xo, 0, xe*1)).
    cos = 1, sin = 0 at pos 1: the head equals the pos-0 result exactly.  A swapped table, a wrong sign or
    a wrong partner index fails one of these."""
    T, H, D = 2, 3, 128
    x = C.normal(3, (T, H, D))
    w = C.norm_weight(4, D)
    n = _normed(oracle, x, w, 1e-6)
    half = D // 2
    c90 = np.zeros((2, half), F)
    s90 = np.zeros((2, half), F)
    c90[1] = 0.0
    s90[1] = 1.0
    got = oracle.rmsnorm_rope(x, w, c90, s90, np.ones(T, np.int32), 1e-6)
    assert bits_equal(got[..., :half], -n[..., half:])
    assert bits_equal(got[..., half:], n[..., :half])
    c0 = np.ones((2, half), F)
    s0 = np.zeros((2, half), F)
    got = oracle.rmsnorm_rope(x, w, c0, s0, np.ones(T, np.int32), 1e-6)
    assert bits_equal(got, n)


def _rn32_exact(v):
    """binary32 nearest-even of a float64 value that holds the exact result."""
    return F(v)


def test_rope_rotation_fused_known_answers(oracle):
    """A head of ones with eps 0 has scale exactly 1, so xe = w_j and xo = w_{j+h} exactly.  With 16-bit
    significands for w and the pos-1 table row, every product is exact in double, so the reference's
    out_j = fma(-xo, sin, RN(xe*cos)) and out_{j+h} = fma(xo, cos, RN(xe*sin)) have closed forms with one
    rounding each.  Unfused rotations, or the FMA on the other product, differ on part of the pairs."""
    D, half = 64, 32
    r = np.random.default_rng(77)
    def v16(n):
        return (r.integers(1 << 15, 1 << 16, n).astype(np.float64) / (1 << 15) * r.choice([-1.0, 1.0], n)).astype(F)
    a, b, c1, s1 = v16(half), v16(half), v16(half), v16(half)
    w = np.concatenate([a, b])
    ct = np.stack([np.ones(half, F), c1])
    st = np.stack([np.zeros(half, F), s1])
    x = np.ones((1, 1, D), F)
    got = oracle.rmsnorm_rope(x, w, ct, st, np.array([1], np.int32), 0.0)[0, 0]
    a64, b64, c64, s64 = (t.astype(np.float64) for t in (a, b, c1, s1))
    re = (a * c1).astype(F).astype(np.float64)  # RN(xe*cos)
    ro = (a * s1).astype(F).astype(np.float64)  # RN(xe*sin)
    want_lo = _rn32_exact(re - b64 * s64)
    want_hi = _rn32_exact(ro + b64 * c64)
    assert bits_equal(got[:half], want_lo) and bits_equal(got[half:], want_hi)
    unfused = (re.astype(F) - (b * s1).astype(F)).astype(F)
    other = _rn32_exact((-(b * s1)).astype(F).astype(np.float64) + a64 * c64)
    assert not bits_equal(unfused, want_lo) and not bits_equal(other, want_lo)


def test_rope_pos0_skips_the_tables(oracle):
    """pos 0 takes the norm-only path whatever the table row 0 holds (here a quarter turn), for RMSNorm+RoPE
    and for RoPE only (which returns the head unchanged)."""
    x = C.normal(9, (1, 3, 64))
    w = C.norm_weight(10, 64)
    ct = np.zeros((1, 32), F)
    st = np.ones((1, 32), F)
    got = oracle.rmsnorm_rope(x, w, ct, st, np.zeros(1, np.int32), 1e-6)
    assert bits_equal(got, _normed(oracle, x, w, 1e-6))
    assert bits_equal(oracle.rope_only(x, ct, st, np.zeros(1, np.int32)), x)


def test_rope_rotation_preserves_pair_norms(oracle):
    T, H, D = 64, 4, 128
    x = C.normal(5, (T, H, D))
    w = C.norm_weight(6, D)
    ct, st = oracle.rope_tables(T, D, 1e6)
    pos = np.arange(T, dtype=np.int32)
    got = oracle.rmsnorm_rope(x, w, ct, st, pos, 1e-6).astype(np.float64)
    n = _normed(oracle, x, w, 1e-6).astype(np.float64)
    h = D // 2
    r_got = np.hypot(got[..., :h], got[..., h:])
    r_n = np.hypot(n[..., :h], n[..., h:])
    assert np.max(np.abs(r_got - r_n) / np.maximum(r_n, 1e-6)) < 1e-6


@pytest.mark.parametrize("heads,hd,pos,eps", [(1, 64, 0, 1e-6), (1, 64, 7, 1e-6), (4, 64, 31, 1e-6),
                                              (8, 128, 0, 1e-6), (16, 64, 31, 1e-6), (32, 128, 0, 1e-6),
                                              (40, 64, 31, 1e-6), (40, 128, 7, 1e-6), (32, 64, 31, 1e-5),
                                              (8, 64, 7, 1e-5)])
@pytest.mark.parametrize("seed", [12345, 67890])
def test_rope_vs_validator_double_ref(oracle, heads, hd, pos, eps, seed):
    """tools/v_rmsnorm_validate.cpp:67-83 cases against the double reference (tools/kt_utils.h:460-485),
    tolerance 1e-3 as the reference validator; also within 2e-5 absolute (outputs are O(1))."""
    buf = C.validator_row(seed, heads * hd).reshape(1, heads, hd)
    w = C.validator_weight(seed + 1, hd)
    ct, st = C.validator_rope_tables(pos, hd, hd)
    got = oracle.rmsnorm_rope(buf, w, ct, st, np.array([pos], np.int32), eps)
    ref = oracle.rmsnorm_rope_double_ref(buf, w, ct, st, [pos], eps)
    assert np.max(np.abs(got - ref)) < 1e-3
    b = buf.astype(np.float64)
    sc = 1.0 / np.sqrt(np.mean(b * b, axis=-1, keepdims=True) + eps)
    xn = b * sc * w
    h = hd // 2
    c = ct[pos, :h].astype(np.float64)
    s = st[pos, :h].astype(np.float64)
    d = np.concatenate([xn[..., :h] * c - xn[..., h:] * s, xn[..., :h] * s + xn[..., h:] * c], axis=-1)
    assert np.max(np.abs(got - d)) < 2e-5


def test_rope_tables_vs_double(oracle):
    """freq_j = base^(-j/half), cos/sin(pos*freq_j) rounded once to binary32: within 1 ulp of numpy double."""
    P, D, base = 2048, 128, 1e6
    c, s = oracle.rope_tables(P, D, base)
    half = D // 2
    f = np.power(np.float64(base), -np.arange(half, dtype=np.float64) / half)
    ang = np.arange(P, dtype=np.float64)[:, None] * f[None, :]
    dc, ds = np.cos(ang), np.sin(ang)
    assert np.all(np.abs(c - dc) <= np.spacing(np.abs(dc).astype(F)) + 1e-12)
    assert np.all(np.abs(s - ds) <= np.spacing(np.abs(ds).astype(F)) + 1e-12)
    assert np.all(c[0] == 1.0) and np.all(s[0] == 0.0)


def test_rope_freqs_x87_chain_closed_forms_and_rounding(oracle):
    """The frequencies come from the reference's x87 chain (fyl2x, frndint, f2xm1, fscale in extended precision,
    src/asm/fused_f32_kernel.inc:117-134) stored as doubles.  Pinned by exact closed forms (a power-of-two base
    with j/half a dyadic fraction gives an exact power of two; j = 0 gives 1) and, for the bases models use, by
    the correctly rounded value of base^(-j/half) from 50-digit decimal arithmetic: a 64-bit-significand chain
    rounded once to double may differ from it by at most one ulp, and rarely does."""
    import decimal

    assert np.array_equal(oracle.rope_freqs(8, 256.0), 2.0 ** -np.arange(8))  # y = -j exactly
    assert np.array_equal(oracle.rope_freqs(2, 4.0), [1.0, 0.5])
    f = oracle.rope_freqs(64, 65536.0)
    assert f[0] == 1.0 and f[16] == 2.0 ** -4 and f[32] == 2.0 ** -8 and f[48] == 2.0 ** -12
    decimal.getcontext().prec = 50
    total = off = 0
    for base in (1e4, 1e5, 5e5, 1e6, 5e6):
        for half in (32, 64, 128):
            got = oracle.rope_freqs(half, base)
            for j in range(half):
                exact = float(decimal.Decimal(base) ** (decimal.Decimal(-j) / decimal.Decimal(half)))
                total += 1
                if got[j] != exact:
                    off += 1
                    assert abs(got[j] - exact) <= np.spacing(exact), (base, half, j)
    assert off <= total // 100, (off, total)


LLAMA31 = dict(base=500000.0, factor=8.0, low=1.0, high=4.0, orig=8192)  # Llama 3.1 8B config.json


def test_rope_llama3_freqs_vs_transformers(oracle):
    """The scaled frequencies equal the library routine transformers.modeling_rope_utils._compute_llama3_parameters
    (torch float32) within its float32 rounding, for the Llama 3.1 8B parameters and for another set."""
    pytest.importorskip("transformers")
    from transformers import LlamaConfig
    from transformers.modeling_rope_utils import _compute_llama3_parameters

    for base, factor, low, high, orig, hd in ((500000.0, 8.0, 1.0, 4.0, 8192, 128), (10000.0, 4.0, 2.0, 8.0, 2048, 64)):
        cfg = LlamaConfig(hidden_size=hd * 8, num_attention_heads=8, max_position_embeddings=4 * orig,
                          rope_parameters={"rope_type": "llama3", "rope_theta": base, "factor": factor,
                                           "low_freq_factor": low, "high_freq_factor": high,
                                           "original_max_position_embeddings": orig})
        inv, _ = _compute_llama3_parameters(cfg, device="cpu")
        want = inv.double().numpy()
        got = oracle.rope_freqs_llama3(hd // 2, base, factor, low, high, orig)
        assert np.max(np.abs(got - want) / want) < 2e-6


def test_rope_llama3_regimes_closed_forms(oracle):
    """High frequencies (wavelength below orig/high) keep base^(-j/half); low frequencies (wavelength above
    orig/low) are divided by factor; the band between interpolates, so it lies between the two; factor 1 is
    the plain table."""
    p = LLAMA31
    half = 64
    plain = np.power(np.float64(p["base"]), -np.arange(half, dtype=np.float64) / half)
    got = oracle.rope_freqs_llama3(half, p["base"], p["factor"], p["low"], p["high"], p["orig"])
    wl = 2 * np.pi / plain
    hi_f, lo_f = wl < p["orig"] / p["high"], wl > p["orig"] / p["low"]
    mid = ~hi_f & ~lo_f
    assert hi_f.any() and lo_f.any() and mid.any()
    assert np.allclose(got[hi_f], plain[hi_f], rtol=4e-16, atol=0)
    assert np.allclose(got[lo_f], plain[lo_f] / p["factor"], rtol=4e-16, atol=0)
    assert np.all(got[mid] <= plain[mid] * (1 + 1e-15)) and np.all(got[mid] >= plain[mid] / p["factor"] * (1 - 1e-15))
    assert np.all(np.diff(got) < 0)  # still strictly decreasing in j
    same = oracle.rope_freqs_llama3(half, p["base"], 1.0, p["low"], p["high"], p["orig"])
    assert np.allclose(same, plain, rtol=4e-16, atol=0)


def test_rope_llama3_tables_vs_double(oracle):
    """cos/sin(pos * freq_j) rounded once to binary32: within 1 ulp of numpy double on the scaled frequencies."""
    p = LLAMA31
    P, D = 1024, 128
    c, s = oracle.rope_tables_llama3(P, D, p["base"], p["factor"], p["low"], p["high"], p["orig"])
    f = oracle.rope_freqs_llama3(D // 2, p["base"], p["factor"], p["low"], p["high"], p["orig"])
    ang = np.arange(P, dtype=np.float64)[:, None] * f[None, :]
    dc, ds = np.cos(ang), np.sin(ang)
    assert np.all(np.abs(c - dc) <= np.spacing(np.abs(dc).astype(F)) + 1e-12)
    assert np.all(np.abs(s - ds) <= np.spacing(np.abs(ds).astype(F)) + 1e-12)


# --------------------------------------------------------------------------- sigmoid / SwiGLU (a5, a6, a8)

def test_sigmoid_constants_and_special_values(oracle):
    assert float(oracle.sigmoid(0.0)) == 0.5  # fx = 0: p = 1, e = 1, 1/(1+1)
    assert float(oracle.sigmoid(100.0)) == 1.0  # clamped to -80: e = 2^-115.4.., 1/(1+e) rounds to 1
    lo = float(oracle.sigmoid(-100.0))  # clamped to 80: 1/(1+e^80)
    assert abs(lo - math.exp(-80.0)) / math.exp(-80.0) < 1e-6
    # vmaxps(NaN, -80) returns -80: a NaN gate clamps to x = -80, i.e. sigmoid 1 (then NaN * 1 in SwiGLU)
    assert float(oracle.sigmoid(float("nan"))) == 1.0


def test_sigmoid_exact_where_the_exponent_is_an_integer(oracle):
    """Inputs g whose fx = RN(-g * log2e) is an integer k leave f = fx - rint(fx) = 0, so the Horner
    polynomial is exactly 1 (every term vanishes) and e = 2^k exactly: the reference's result is then
    RN(1 / RN(1 + 2^k)), a closed form.  This pins the steps around the polynomial bit for bit: the
    negation, the exponent built from k, the 1 + e and the final reciprocal (a swapped sign or e/(1+e)
    for 1/(1+e) fails here; floor for rint, a contracted fx - rint(fx) or a misplaced coefficient fail
    the dense sweep below)."""
    log2e = F(1.4426950408889634)
    checked = 0
    for k in range(-23, 24):
        y = F(k / 1.4426950408889634)
        for _ in range(8):  # nearest float32 y with RN(y * log2e) == k
            if F(y * log2e) == F(k):
                break
            y = np.nextafter(y, F(np.inf) if F(y * log2e) < k else F(-np.inf), dtype=F)
        if F(y * log2e) != F(k):
            continue
        g = float(-y)
        want = F(1.0) / (F(1.0) + F(2.0 ** k))  # 1 + 2^k is exact for |k| <= 23
        assert bits_equal(np.array([oracle.sigmoid(g)], F), np.array([want], F)), (k, g)
        checked += 1
    assert checked >= 40


def test_sigmoid_dense_sweep_vs_double(oracle):
    """The degree-5 exp2 polynomial is stated at 1.27e-7 max relative error (src/asm/v7_macros.inc:127-128).
    With the roundings around it the sigmoid stays within 5e-7 relative of double, plus the error that the
    rounding of fx = -g*log2e carries into 2^fx for g < 0 (half an ulp of |fx|, times ln 2: about
    6e-8 * |g|).  A wrong coefficient or a misplaced Horner operand breaks this by orders of magnitude."""
    g = np.linspace(-80.0, 30.0, 400001).astype(F)
    got = np.array([oracle.sigmoid(float(v)) for v in g[::7]], np.float64)
    gd = g[::7].astype(np.float64)
    ref = 1.0 / (1.0 + np.exp(-gd))
    rel = np.abs(got - ref) / ref
    assert np.all(rel < 5e-7 + 7e-8 * np.maximum(-gd, 0.0))
    assert np.max(rel[gd > -4]) < 5e-7


def test_swiglu_vs_double(oracle):
    g = C.normal(301, 200000, 1.5)
    u = C.normal(302, 200000, 1.5)
    got = oracle.swiglu(g, u).astype(np.float64)
    ref = g.astype(np.float64) / (1.0 + np.exp(-g.astype(np.float64))) * u
    m = np.abs(ref) > 1e-30
    assert np.max(np.abs(got - ref)[m] / np.abs(ref)[m]) < 1e-5
    # u = 1 leaves silu(g) = sigmoid(g)*g, one binary32 multiply after the sigmoid
    gs = C.normal(7, 1000, 1.5)
    sil = np.array([np.float32(oracle.sigmoid(float(v))) * v for v in gs], F)
    assert bits_equal(oracle.swiglu(gs, np.ones_like(gs)), sil)


# --------------------------------------------------------------------------- quantize (a7) and SwiGLU -> Q8 (a8)

def test_quantizer_floor_constant():
    """scalar_epsilon = 127 * 2^-126 (src/asm/quantize_kernel.inc:40-41): its /127 is exactly 2^-126."""
    fl = np.float32(1.4928778e-36)
    assert fl == np.float32(127.0) * np.float32(2.0 ** -126)
    assert fl / np.float32(127.0) == np.float32(2.0 ** -126)


@pytest.mark.parametrize("pattern", C.KT_PATTERNS)
@pytest.mark.parametrize("n", [64, 256, 1024, 4096, 8192, 65536])
def test_quantize_vs_kt_quantize_c_ref(oracle, pattern, n):
    """tools/v_quantize_validate.cpp: 7 patterns x sizes x seeds {12345, 67890, 11111}; int8 codes must equal
    kt_quantize_c_ref's exactly; scales equal except the all-zero group (1/127 there, 2^-126 in the kernel)."""
    for seed in (12345, 67890, 11111):
        x = C.kt_pattern(pattern, n, seed)
        q, s = oracle.quantize(x[None], 64)
        kq, ks = oracle.kt_quantize_c_ref(x)
        assert bits_equal(q[0], kq), pattern
        nz = np.max(np.abs(x.reshape(-1, 64)), axis=1) > 0
        assert bits_equal(s[0][nz], ks[nz])
        assert np.all(s[0][~nz] == np.float32(2.0 ** -126))


@pytest.mark.parametrize("gs", [32, 64])
def test_quantize_closed_form_properties(oracle, gs):
    x = C.normal(9, (37, 1024), 2.0)
    x[3, :gs] = 0.0
    q, s = oracle.quantize(x, gs)
    xg = x.reshape(37, -1, gs).astype(np.float64)
    qg = q.reshape(37, -1, gs).astype(np.float64)
    amax = np.max(np.abs(xg), axis=-1)
    assert np.all(s[amax > 0] == (amax[amax > 0] / 127.0).astype(F)) or np.allclose(
        s[amax > 0], amax[amax > 0] / 127.0, rtol=6e-8)
    # the group's largest magnitude maps to +-127; every code within half a step (plus rounding) of x/scale
    assert np.all(np.max(np.abs(qg), axis=-1)[amax > 0] == 127)
    err = np.abs(xg - qg * s[..., None].astype(np.float64))
    assert np.all(err <= 0.5 * s[..., None] * (1 + 1e-5))
    assert np.all(qg[3, 0] == 0) and s[3, 0] == np.float32(2.0 ** -126)
    assert q.min() >= -127


def test_quantize_tail_group(oracle):
    """n % gs != 0: the last, partial group uses the scalar tail (quantize_kernel.inc:119-152) -- the same
    values as quantizing that partial group on its own."""
    x = C.normal(11, 100, 3.0)
    q, s = oracle.quantize(x[None], 64)
    q1, s1 = oracle.quantize(x[None, :64], 64)
    q2, s2 = oracle.quantize(x[None, 64:], 64)
    assert bits_equal(q[0], np.concatenate([q1[0], q2[0]]))
    assert bits_equal(s[0], np.concatenate([s1[0], s2[0]]))
    kq, _ = oracle.kt_quantize_c_ref(x)
    assert bits_equal(q[0], kq)


def test_quantize_ties_to_even_and_nan_codes(oracle):
    """A group whose absmax is 127 has scale exactly 1 and reciprocal 1, so its codes are the nearest-even
    integers of the inputs: vcvtps2dq on full groups and the tail's vcvtss2si both round ties to even
    (2.5 -> 2, -3.5 -> -4, 0.5 -> 0, 126.5 -> 126).  A NaN element becomes -128 after the saturating packs
    and -127 after vpmaxsb (full group), or -127 from the tail's vmaxss; a separately rounded tail or a
    code left at -128 fails here."""
    vals = np.array([127.0, 2.5, -3.5, 0.5, -0.5, 126.5], F)
    want = np.array([127, 2, -4, 0, 0, 126], np.int8)
    x = np.zeros(70, F)  # one full group of 64, then a 6-element tail
    x[:6] = vals
    x[64:] = vals
    q, sc = oracle.quantize(x[None], 64)
    assert sc[0, 0] == 1.0 and sc[0, 1] == 1.0
    assert bits_equal(q[0, :6], want) and bits_equal(q[0, 64:], want) and not q[0, 6:64].any()
    y = x.copy()
    y[0] = np.nan  # absmax of the rest is still 127 (the NaN lane drops out of the max tree first)
    y[1] = 127.0
    y[64 + 5] = np.nan
    q, _ = oracle.quantize(y[None], 64)
    assert q[0, 0] == -127 and q[0, 64 + 5] == -127


def test_quantize_nan_position_in_the_max_tree(oracle):
    """vmaxps returns its second operand when either is NaN, so the group max of the vector path depends
    on where a NaN sits (src/asm/quantize_kernel.inc:62-84 and the note at :128).  Hand-traced cases:
    - NaN at element 63 (vector 7, lane 7) is the second operand at every level of the tree: wmax is NaN,
      vmaxss wmax, eps gives the floor 127*2^-126, scale 2^-126, reciprocal 2^126.  Codes are then
      rne(x * 2^126) saturated: 3*2^-126 -> 3, 2^-120 -> 64, 2^-100 -> 127, -2^-100 -> -127, and
      2^-94 or 1.0 -> -127 (beyond 2^31 vcvtps2dq gives 0x80000000, whatever the sign);
    - the same for element 31 of a 32-element group (vector 3, lane 7);
    - NaN at element 62 (lane 6) reaches vmaxps(p0, p2) as p2 and then is the first operand of the last
      vmaxps: it drops out, wmax = 1;
    - NaN at element 8 (vector 1, lane 0) survives vmaxps(v0, v1) and drops out at the next level, taking
      element 0 with it: wmax = 1 although x[0] = 2^40, whose code is then -127;
    - NaN at element 16 (vector 2) is the first operand of vmaxps(v2, v3) and drops out alone: wmax is
      x[0] = 2^40 (an in-order scan of the vectors would have lost it);
    - the scalar tail (vmaxss |x|, wmax) and the in-order scan of other group sizes always drop a NaN."""
    tiny = np.array([3 * 2.0 ** -126, 2.0 ** -120, 2.0 ** -100, -2.0 ** -100, 2.0 ** -94, 0.0, 1.0], F)
    tiny_codes = np.array([3, 64, 127, -127, -127, 0, -127], np.int8)
    for gs, at in ((64, 63), (32, 31)):
        x = np.ones(gs, F)
        x[:7] = tiny
        x[at] = np.nan
        q, s = oracle.quantize(x[None], gs)
        assert s[0, 0] == np.float32(2.0 ** -126)
        assert bits_equal(q[0, :7], tiny_codes) and np.all(q[0, 7:] == -127)
    one_127 = np.float32(1.0) / np.float32(127.0)
    x = np.ones(64, F)
    x[62] = np.nan
    q, s = oracle.quantize(x[None], 64)
    assert s[0, 0] == one_127 and q[0, 62] == -127 and np.all(np.delete(q[0], 62) == 127)
    for gs in (64, 32):
        x = np.ones(gs, F)
        x[0] = 2.0 ** 40
        x[8] = np.nan
        q, s = oracle.quantize(x[None], gs)
        assert s[0, 0] == one_127 and q[0, 0] == -127 and q[0, 8] == -127
        assert np.all(np.delete(q[0], [0, 8]) == 127)
        x[8] = 1.0
        x[16] = np.nan
        q, s = oracle.quantize(x[None], gs)
        assert s[0, 0] == np.float32(2.0 ** 40) / np.float32(127.0) and q[0, 0] == 127 and q[0, 16] == -127
        assert np.all(np.delete(q[0], [0, 16]) == 0)
    x = np.ones(16, F)
    x[15] = np.nan
    x[3] = 2.0
    q, s = oracle.quantize(x[None], 16)
    assert s[0, 0] == np.float32(2.0) / np.float32(127.0) and q[0, 3] == 127 and q[0, 15] == -127
    x = np.ones(64 + 10, F)
    x[-1] = np.nan
    q, s = oracle.quantize(x[None], 64)
    assert s[0, 1] == one_127 and q[0, -1] == -127 and np.all(q[0, 64:-1] == 127)


def test_swiglu_q8_is_quantize_of_swiglu_and_near_double(oracle):
    g = C.normal(401, (16, 8192), 1.5)
    u = C.normal(402, (16, 8192), 1.5)
    for gs in (32, 64):
        q, s = oracle.swiglu_q8(g, u, gs)
        q2, s2 = oracle.quantize(oracle.swiglu(g, u), gs)
        assert bits_equal(q, q2) and bits_equal(s, s2)
        ref = (g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64))) * u).reshape(16, -1, gs)
        ideal = ref / s[..., None].astype(np.float64)
        assert np.max(np.abs(q.reshape(16, -1, gs) - ideal)) <= 0.5 + 1e-3


# --------------------------------------------------------------------------- FP environment: MXCSR FTZ + DAZ

avx2_early = pytest.mark.skipif("not __import__('oracle.oracle', fromlist=['x']).avx2_available()",
                                reason="host CPU lacks AVX2/FMA")


def test_oracle_runs_in_the_reference_fp_environment(oracle):
    """The reference computes under MXCSR FTZ+DAZ (src/asm/v7_init.inc:103-108, SET_FTZ_DAZ
    src/asm/v7_core.inc:301-303): a denormal input reads as zero and a result still below 2^-126 after
    rounding becomes zero.  Hand-traced cases, each also run with gradual underflow to show the switch
    is what decides them:
    - quantize, x = [2^-120, 1.5*2^-127, 0...]: wmax 2^-120 is below the floor, so scale 2^-126 and
      reciprocal 2^126; 2^-120 -> 64; the denormal reads as 0 -> code 0 (gradual underflow: 0.75 -> 1);
    - RMSNorm, 64 x 2^-70, w = 1, eps = 0: every square 2^-140 flushes, sumsq = 0, scale = 1/sqrt(0) = Inf,
      o = Inf (gradual underflow: sumsq 2^-134, mean 2^-140, scale 2^70, o = 1);
    - SwiGLU, g = 2^-130, u = 1: the clamp reads g as 0, sigmoid = 1/(1+1) = 0.5, sigma*g = 0.5*0 = 0
      (gradual underflow: 2^-131);
    - add, 2^-127 + 2^-127 = 0 (gradual underflow: 2^-126); 1.5*2^-126 - 2^-126, two normal inputs whose
      sum 2^-127 flushes = 0 (gradual underflow, or DAZ alone: 2^-127);
    - RMSNorm+RoPE at pos 0 of a head of 64 x 2^-127, eps 1e-6: x reads as 0, so every output is 0
      (gradual underflow: x * 1/sqrt(eps) is about 2^-117)."""
    d = np.float32(2.0 ** -127) * np.float32(1.5)
    xq = np.zeros((1, 64), F)
    xq[0, 0] = 2.0 ** -120
    xq[0, 1] = d
    x70 = np.full((1, 64), 2.0 ** -70, F)
    g = np.array([2.0 ** -130], F)
    a = np.array([2.0 ** -127], F)
    head = np.full((1, 1, 64), 2.0 ** -127, F)
    ct, st = oracle.rope_tables(1, 64, 1e6)
    pos = np.zeros(1, np.int32)

    def run():
        q, s = oracle.quantize(xq, 64)
        return (q[0, :2].tolist(), float(s[0, 0]), float(oracle.rmsnorm(x70, np.ones(64, F), 0.0)[0, 0]),
                float(oracle.swiglu(g, np.ones(1, F))[0]), float(oracle.add_inplace(a, a)[0]),
                float(oracle.add_inplace(np.array([1.5 * 2.0 ** -126], F), np.array([-2.0 ** -126], F))[0]),
                float(np.max(np.abs(oracle.rmsnorm_rope(head, np.ones(64, F), ct, st, pos, 1e-6)))))

    assert oracle.lib().orc_get_reference_fp_env() == 1
    q, s, o, sw, ad, ad2, rope = run()
    assert q == [64, 0] and s == 2.0 ** -126
    assert o == np.inf and sw == 0.0 and ad == 0.0 and ad2 == 0.0 and rope == 0.0
    with oracle.gradual_underflow():
        q, s, o, sw, ad, ad2, rope = run()
    assert q == [64, 1] and s == 2.0 ** -126
    assert o == 1.0 and sw == 2.0 ** -131 and ad == 2.0 ** -126 and ad2 == 2.0 ** -127 and 0 < rope < 2.0 ** -100
    assert oracle.lib().orc_get_reference_fp_env() == 1


@avx2_early
def test_avx2_form_matches_scalar_oracle_on_denormal_data(oracle):
    """Both restatements in the reference's FTZ+DAZ mode agree bit for bit on data full of denormals and
    tiny values (the AVX2 form runs the same vector instructions as the reference)."""
    rng = C.rng(71)
    bits = rng.integers(0, 0x00800000, (8, 4096), dtype=np.uint32) | (rng.integers(0, 2, (8, 4096), dtype=np.uint32) << 31)
    x = bits.view(F).copy()
    x[:, ::3] = C.normal(72, (8, 4096))[:, ::3] * np.float32(2.0 ** -60)
    x[:, ::7] = C.normal(73, (8, 4096))[:, ::7]
    y = x[::-1].copy()
    w = C.norm_weight(74, 4096)
    assert all(bits_equal(p, q) for p, q in zip(oracle.avx2_fused_add_rmsnorm_rows(x, y, w, 0.0),
                                                 oracle.fused_add_rmsnorm(x, y, w, 0.0)))
    assert bits_equal(oracle.avx2_swiglu(x.reshape(-1), y.reshape(-1)), oracle.swiglu(x.reshape(-1), y.reshape(-1)))
    for gs in (32, 64):
        assert all(bits_equal(p, q) for p, q in zip(oracle.avx2_quantize(x, gs), oracle.quantize(x, gs)))
    h = x.reshape(8, 32, 128)
    ct, st = oracle.rope_tables(8, 128, 1e6)
    pos = np.arange(8, dtype=np.int32)
    assert bits_equal(oracle.avx2_rmsnorm_rope(h, w[:128], ct, st, pos, 1e-6),
                      oracle.rmsnorm_rope(h, w[:128], ct, st, pos, 1e-6))


# --------------------------------------------------------------------------- embedding dequant (a9)

def test_embedding_closed_form(oracle):
    """out[i] = (float)q[token*dim + i] * s[(token*dim)/64 + i/64] (src/asm/forward.inc:13-42): exact convert,
    one binary32 multiply."""
    vocab, dim = 300, 256
    tq, ts = C.q8_table(21, vocab, dim)
    ids = C.rng(22).integers(0, vocab, 50).astype(np.int32)
    got = oracle.embedding_gather(ids, tq, ts, dim)
    want = tq[ids].astype(F) * np.repeat(ts.reshape(vocab, dim // 64)[ids], 64, axis=1)
    assert bits_equal(got, want.astype(F))


# --------------------------------------------------------------------------- AVX2 restatement (CPU baseline)

avx2 = pytest.mark.skipif("not __import__('oracle.oracle', fromlist=['x']).avx2_available()",
                          reason="host CPU lacks AVX2/FMA")


@avx2
def test_avx2_matches_scalar_oracle(oracle):
    r = C.normal(1, (8, 4096))
    a = C.normal(2, (8, 4096))
    w = C.norm_weight(3, 4096)
    assert all(bits_equal(p, q) for p, q in zip(oracle.avx2_fused_add_rmsnorm_rows(r, a, w, 1e-6),
                                                 oracle.fused_add_rmsnorm(r, a, w, 1e-6)))
    for dim in (8, 24, 40, 72):
        r2, a2, w2 = C.normal(dim, (3, dim)), C.normal(dim + 1, (3, dim)), C.norm_weight(dim, dim)
        assert all(bits_equal(p, q) for p, q in zip(oracle.avx2_fused_add_rmsnorm_rows(r2, a2, w2, 1e-5),
                                                     oracle.fused_add_rmsnorm(r2, a2, w2, 1e-5)))
    x = C.normal(4, (16, 8, 128))
    qw = C.norm_weight(5, 128)
    ct, st = oracle.rope_tables(16, 128, 1e6)
    pos = np.arange(16, dtype=np.int32)
    assert bits_equal(oracle.avx2_rmsnorm_rope(x, qw, ct, st, pos, 1e-6), oracle.rmsnorm_rope(x, qw, ct, st, pos, 1e-6))
    g = C.normal(6, 100003, 1.5)
    u = C.normal(7, 100003, 1.5)
    assert bits_equal(oracle.avx2_swiglu(g, u), oracle.swiglu(g, u))
    xq = C.normal(8, (5, 8192 + 40), 2.0)
    for gs in (32, 64):
        assert all(bits_equal(p, q) for p, q in zip(oracle.avx2_quantize(xq, gs), oracle.quantize(xq, gs)))
    # NaN sprinkled over the groups: the hardware vmaxps of the AVX2 form against the scalar tree
    xn = xq.copy()
    pick = C.rng(11).integers(0, xn.size, 600)
    xn.reshape(-1)[pick] = np.nan
    xn.reshape(-1)[pick[:200] + 1] = C.rng(12).uniform(1e3, 1e12, 200).astype(F)
    for gs in (32, 64):
        assert all(bits_equal(p, q) for p, q in zip(oracle.avx2_quantize(xn, gs), oracle.quantize(xn, gs)))
    tq, ts = C.q8_table(9, 100, 512)
    ids = C.rng(10).integers(0, 100, 20).astype(np.int32)
    assert bits_equal(oracle.avx2_embedding_gather(ids, tq, ts, 512), oracle.embedding_gather(ids, tq, ts, 512))
    # RMSNorm alone (leftover 8-float blocks included) and vaddps, used by the widened rows' timing driver
    L = oracle.lib()
    for dim in (8, 40, 256, 4096):
        xr, wr = C.normal(dim + 2, dim), C.norm_weight(dim + 3, dim)
        got = np.empty(dim, F)
        L.orc_avx2_rmsnorm(got.ctypes.data_as(ctypes.c_void_p), xr.ctypes.data_as(ctypes.c_void_p),
                           wr.ctypes.data_as(ctypes.c_void_p), dim, ctypes.c_float(1e-6))
        assert bits_equal(got, oracle.rmsnorm(xr[None], wr, 1e-6)[0])
    xa, ya = C.normal(13, 1003), C.normal(14, 1003)
    got = xa.copy()
    L.orc_avx2_add_inplace(got.ctypes.data_as(ctypes.c_void_p), ya.ctypes.data_as(ctypes.c_void_p),
                           ctypes.c_longlong(1003))
    assert bits_equal(got, oracle.add_inplace(xa, ya))
    # RoPE without the norm (rope_only_kernel.inc's vmulps / vfnmadd231ps / vfmadd231ps order) against the
    # scalar restatement, at every head_dim class, position 0 (no rotation) and the last table row
    for hd in (64, 96, 128, 256, 512):
        ct, st = oracle.rope_tables(40, hd, 1e4)
        for pos in (0, 1, 17, 39):
            x = C.normal(hd + pos, (5, hd))
            want, got = x.copy(), x.copy()
            L.orc_rope_only_heads(want, 5, hd, ct, st, pos, hd // 2)
            L.orc_avx2_rope_only_heads(got, 5, hd, ct, st, pos, hd // 2)
            assert bits_equal(got, want), (hd, pos)
            assert pos > 0 or bits_equal(got, x)


# --------------------------------------------------------------------------- next rows: rmsnorm, rmsnorm_quantize, add_inplace

RMS_SIZES = [64, 128, 256, 1024, 2048, 3072, 8192]  # tools/v_rmsnorm_validate.cpp:51-61


@pytest.mark.parametrize("size", RMS_SIZES)
@pytest.mark.parametrize("seed", [12345, 67890])
def test_rmsnorm_vs_validator_refs(oracle, size, seed):
    """v7s_rmsnorm against the float C reference (tools/kt_utils.h:450-458) within 1e-3, the validator's
    tolerance (tools/kt_utils.h:820), and against double precision within 1e-5 relative."""
    x = C.validator_row(seed, size)
    w = C.validator_weight(seed + 1, size)
    o = oracle.rmsnorm(x[None], w, 1e-6)[0]
    assert np.max(np.abs(o - oracle.kt_rmsnorm_c_ref(x, w, 1e-6))) < 1e-3
    xd = x.astype(np.float64)
    d = xd / np.sqrt(np.mean(xd * xd) + 1e-6) * w
    assert np.max(np.abs(o - d) / np.maximum(np.abs(d), 1e-3)) < 1e-5


def test_rmsnorm_order_matches_add_rmsnorm_and_known_answer(oracle):
    """The two kernels accumulate in the same order for size % 32 == 0 (src/asm/rmsnorm_kernel.inc:22-48 and
    add_rmsnorm_kernel.inc:29-73): with add = 0 the residual is unchanged and the outputs agree bit for bit.
    Known answer: the accumulator-interleave input of the sum-of-squares test (sumsq 2^24 + 4) normalised with
    w = 1 and eps = 0 scales by 1/sqrt((2^24 + 4)/64)."""
    x = C.normal(77, (4, 1024))
    w = C.norm_weight(78, 1024)
    o, r = oracle.fused_add_rmsnorm(x, np.zeros_like(x), w, 1e-6)
    assert bits_equal(r, x) and bits_equal(oracle.rmsnorm(x, w, 1e-6), o)
    k = np.zeros(64, F)
    k[0] = 4096.0
    for i in (8, 16, 24, 32, 40):
        k[i] = 1.0
    s = F(1.0) / np.sqrt(F(F(TWO24 + 4) / F(64)))
    assert bits_equal(oracle.rmsnorm(k[None], np.ones(64, F), 0.0)[0], (s * k).astype(F))


@pytest.mark.parametrize("size", [64, 128, 256, 512, 1024, 2048, 3072, 8192])
@pytest.mark.parametrize("seed", [12345, 67890])
def test_rmsnorm_quantize_is_the_two_step_chain(oracle, size, seed):
    """tools/kt_utils.h:850-933: v7s_rmsnorm_quantize must be bit-identical to v7s_rmsnorm -> v7d_quantize,
    and close to the C-reference chain (non-FMA rounding may move a code by one)."""
    x = C.validator_row(seed, size)
    w = C.validator_weight(seed + 1, size)
    q, s = oracle.rmsnorm_quantize(x[None], w, 1e-6, 64)
    q2, s2 = oracle.quantize(oracle.rmsnorm(x[None], w, 1e-6), 64)
    assert bits_equal(q, q2) and bits_equal(s, s2)
    cq, _ = oracle.kt_quantize_c_ref(oracle.kt_rmsnorm_c_ref(x, w, 1e-6))
    assert np.max(np.abs(q[0].astype(int) - cq.astype(int))) <= 1


def test_add_inplace_exact(oracle):
    """v7s_add_inplace: one binary32 add per element (tools/kt_utils.h:487-491, validator tolerance 1e-6)."""
    for n in (32, 64, 96, 160, 2048):  # tools/v_add_inplace_validate.cpp:21
        x = C.validator_row(n, n)
        y = C.validator_row(n + 1, n)
        assert bits_equal(oracle.add_inplace(x, y), (x + y).astype(F))


# --------------------------------------------------------------------------- v7s_kv_pack_f16

f16c = pytest.mark.skipif("not __import__('oracle.oracle', fromlist=['x']).f16c_available()",
                          reason="host CPU lacks F16C")


@f16c
def test_f16_conversion_exhaustive_vs_f16c(oracle):
    """orc_f32_to_f16_bits equals vcvtps2ph with imm 0 -- the instruction src/asm/kv_f16c.inc uses -- for
    every one of the 2^32 binary32 bit patterns, NaNs included."""
    import os
    threads = max(1, min(16, len(os.sched_getaffinity(0))))
    assert oracle.check_f16_vs_f16c(0, 1 << 32, threads) == 0


def test_kv_pack_f16_vs_numpy_and_f16c(oracle):
    """numpy's float32 -> float16 cast is IEEE round-to-nearest-even: equal bit patterns on finite values,
    overflow to Inf, binary16 subnormals and signed zeros."""
    x = np.concatenate([C.normal(5, 4096, 3.0), C.normal(6, 1024, 3000.0), C.normal(7, 1024, 1e-5),
                        np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, -65520.0, 1e30, 2.0 ** -24, 2.0 ** -25,
                                  3 * 2.0 ** -26, 2.0 ** -14 - 2.0 ** -25, np.inf, -np.inf], F)]).astype(F)
    x = x[: (x.size // 8) * 8]
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert bits_equal(oracle.kv_pack_f16(x), want)
    if oracle.f16c_available():
        assert bits_equal(oracle.avx2_kv_pack_f16(x), want)


# --------------------------------------------------------------------------- RoPE-only heads, QKV bias

def test_rope_only_known_answers(oracle):
    """pos 0: unchanged; quarter-turn tables: (lo, up) -> (-up, lo) exactly; identity tables: unchanged; and the
    rotation equals RMSNorm+RoPE's rotation applied to an already-normalised head (w = 1, scale exactly 1)."""
    T, H, D = 3, 2, 128
    x = C.normal(1, (T, H, D))
    ct, st = oracle.rope_tables(8, D, 1e4)
    assert bits_equal(oracle.rope_only(x, ct, st, np.zeros(T, np.int32)), x)
    half = D // 2
    c90 = np.zeros((2, half), F)
    s90 = np.ones((2, half), F)
    got = oracle.rope_only(x, c90, s90, np.ones(T, np.int32))
    assert bits_equal(got[..., :half], -x[..., half:]) and bits_equal(got[..., half:], x[..., :half])
    got = oracle.rope_only(x, np.ones((2, half), F), np.zeros((2, half), F), np.ones(T, np.int32))
    assert bits_equal(got, x)
    # a head whose sum of squares is exactly D (entries +-1) has scale 1/sqrt(1 + 0) = 1 with eps = 0
    u = np.where(C.normal(2, (T, H, D)) > 0, 1.0, -1.0).astype(F)
    pos = np.array([1, 5, 7], np.int32)
    assert bits_equal(oracle.rope_only(u, ct, st, pos), oracle.rmsnorm_rope(u, np.ones(D, F), ct, st, pos, 0.0))


def test_rope_only_fused_known_answers(oracle):
    """With 16-bit significands for the head and the pos-1 table row every product is exact in double:
    out_j = fma(-up, sin, RN(lo*cos)) and out_{j+h} = fma(up, cos, RN(lo*sin)) each round once."""
    D, half = 64, 32
    r = np.random.default_rng(78)
    def v16(n):
        return (r.integers(1 << 15, 1 << 16, n).astype(np.float64) / (1 << 15) * r.choice([-1.0, 1.0], n)).astype(F)
    lo, up, c1, s1 = v16(half), v16(half), v16(half), v16(half)
    x = np.concatenate([lo, up])[None, None, :]
    ct = np.stack([np.ones(half, F), c1])
    st = np.stack([np.zeros(half, F), s1])
    got = oracle.rope_only(x, ct, st, np.array([1], np.int32))[0, 0]
    re = (lo * c1).astype(F).astype(np.float64)
    ro = (lo * s1).astype(F).astype(np.float64)
    want_lo = F(re - up.astype(np.float64) * s1.astype(np.float64))
    want_hi = F(ro + up.astype(np.float64) * c1.astype(np.float64))
    assert bits_equal(got[:half], want_lo) and bits_equal(got[half:], want_hi)
    assert not bits_equal((re.astype(F) - (up * s1).astype(F)).astype(F), want_lo)


def test_rope_only_vs_double(oracle):
    T, H, D = 16, 4, 128
    x = C.normal(3, (T, H, D))
    ct, st = oracle.rope_tables(T, D, 1e6)
    pos = np.arange(T, dtype=np.int32)
    got = oracle.rope_only(x, ct, st, pos).astype(np.float64)
    c = ct[pos].astype(np.float64)[:, None, :]
    s = st[pos].astype(np.float64)[:, None, :]
    lo, up = x[..., :D // 2].astype(np.float64), x[..., D // 2:].astype(np.float64)
    d = np.concatenate([lo * c - up * s, lo * s + up * c], axis=-1)
    assert np.max(np.abs(got - d)) < 1e-5


def test_bias_add_exact(oracle):
    x = C.normal(4, (5, 1024))
    b = C.normal(5, 1024)
    assert bits_equal(oracle.bias_add(x, b), (x + b).astype(F))


@pytest.mark.parametrize("kind", range(6))
def test_rows_driver_matches_the_per_function_oracle(oracle, kind):
    """The per-row timing driver of the benchmark's CPU leg (orc_rows_bench, oracle/v7_oracle_rows.c) computes
    each widened row exactly as the oracle's own functions do: RMSNorm -> Q8, add then RMSNorm -> Q8, the K/V
    pack, the Q/K/V stage, QKV bias + RoPE only, add_inplace (13 tokens over 3 threads)."""
    import ctypes

    import bench

    T, DIM, NQ, NKV, HD, GS, EPS = 13, 256, 4, 2, 64, 64, 1e-6
    QKV, KVD = (NQ + 2 * NKV) * HD, NKV * HD
    x, add = C.normal(1, (T, DIM)), C.normal(2, (T, DIM))
    w = C.norm_weight(3, DIM)
    qkv = C.normal(4, (T, QKV))
    bias = C.normal(5, QKV, 0.5)
    q_w, k_w = C.norm_weight(6, HD), C.norm_weight(7, HD)
    ct, st = oracle.rope_tables(T + 3, HD, 1e6)
    pos = (np.arange(T) + 2).astype(np.int32)
    pos[4] = 0
    b = dict(x=x.copy(), add=add, w=w, qkv=qkv.copy(), bias=bias, q_w=q_w, k_w=k_w, ct=ct, st=st, pos=pos,
             codes=np.zeros((T, DIM), np.int8), scales=np.zeros((T, DIM // GS), np.float32),
             kc=np.zeros((T, KVD), np.uint16), vc=np.zeros((T, KVD), np.uint16))
    p = lambda a: a.ctypes.data  # noqa: E731
    a = bench.RowsArgs(kind, T, DIM, GS, NQ, NKV, HD, HD // 2, EPS, p(b["x"]), p(b["add"]), p(b["w"]),
                       p(b["codes"]), p(b["scales"]), p(b["qkv"]), QKV, p(b["q_w"]), p(b["k_w"]), p(b["bias"]),
                       p(b["ct"]), p(b["st"]), p(b["pos"]), p(b["kc"]), p(b["vc"]))
    L = oracle.lib()
    L.orc_rows_bench.restype = ctypes.c_double
    L.orc_rows_bench.argtypes = [ctypes.POINTER(bench.RowsArgs), ctypes.c_int, ctypes.c_int, ctypes.c_int]
    assert L.orc_rows_bench(ctypes.byref(a), 1, 3, 1) >= 0
    q3 = lambda r: r[:, :NQ * HD].reshape(T, NQ, HD)  # noqa: E731
    k3 = lambda r: r[:, NQ * HD:(NQ + NKV) * HD].reshape(T, NKV, HD)  # noqa: E731
    v3 = lambda r: r[:, (NQ + NKV) * HD:].reshape(T, NKV, HD)  # noqa: E731
    if kind in (0, 1):
        xs = oracle.add_inplace(x, add) if kind == 1 else x
        wq, ws = oracle.rmsnorm_quantize(xs, w, EPS, GS)
        assert bits_equal(b["x"], xs) and np.array_equal(b["codes"], wq) and bits_equal(b["scales"], ws)
    elif kind == 2:
        assert np.array_equal(b["kc"], oracle.kv_pack_f16(k3(qkv)).reshape(T, KVD))
        assert np.array_equal(b["vc"], oracle.kv_pack_f16(v3(qkv)).reshape(T, KVD))
    elif kind == 3:
        wq, wk, wv, wkc, wvc = oracle.qkv_stage(q3(qkv), k3(qkv), v3(qkv), q_w, k_w, None, None, None, ct, st, pos,
                                                EPS)
        assert bits_equal(q3(b["qkv"]), wq) and bits_equal(k3(b["qkv"]), wk)
        assert np.array_equal(b["kc"], wkc.reshape(T, KVD)) and np.array_equal(b["vc"], wvc.reshape(T, KVD))
    elif kind == 4:
        wq, wk, wv, _, _ = oracle.qkv_stage(q3(qkv), k3(qkv), v3(qkv), None, None, bias[:NQ * HD],
                                            bias[NQ * HD:(NQ + NKV) * HD], bias[(NQ + NKV) * HD:], ct, st, pos, EPS)
        assert bits_equal(q3(b["qkv"]), wq) and bits_equal(k3(b["qkv"]), wk) and bits_equal(v3(b["qkv"]), wv)
    else:
        assert bits_equal(b["x"], oracle.add_inplace(x, add))
