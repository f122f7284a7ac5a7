"""Python bindings of the CPU oracle (test infrastructure only).

Only the test suite, ``__graft_entry__.smoke()`` and the CPU-baseline leg of
``bench.py`` import this module; the product (``v7multiplikator_amd``) never
does.  The C restatement lives in ``v7_oracle.c`` (scalar) and
``v7_oracle_avx2.c`` (AVX2, the CPU baseline); ``v7_oracle_rows.c`` drives
the widened rows per token row for the baseline's timing; ``make -C oracle``
builds ``liboracle.so``.

Besides the lane-faithful restatements, this module holds double-precision
references restating the reference's own C checkers in ``tools/kt_utils.h``
(``kt_quantize_c_ref`` :378-407, ``v7s_rmsnorm_rope_heads_c_ref`` :460-485,
``v7s_fused_add_rmsnorm_c_ref`` :493-503) -- the checks the reference's
validators apply to its NASM kernels.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# V7G_ORACLE_LIB points the tests at another build of the same sources: the mutation check
# (tests/test_oracle_mutations.py) builds copies with one planted mistake each.
_LIB_PATH = os.environ.get("V7G_ORACLE_LIB") or os.path.join(_HERE, "liboracle.so")
_lib = None

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(np.int8, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")


def lib():
    """Loads liboracle.so (built by ``make -C oracle``)."""
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"{_LIB_PATH} is missing: run `make -C oracle`")
        L = ctypes.CDLL(_LIB_PATH)
        c_int, c_ll, c_float = ctypes.c_int, ctypes.c_longlong, ctypes.c_float
        sig = {
            "orc_sumsq_lanes": (c_float, [_f32p, c_int]),
            "orc_rms_scale": (c_float, [c_float, c_int, c_float]),
            "orc_fused_add_rmsnorm_rows": (None, [_f32p, _f32p, _f32p, _f32p, c_int, c_int, c_float]),
            "orc_rmsnorm_rope_tokens": (None, [_f32p, c_int, c_ll, c_int, c_int, _f32p, _f32p, _f32p, _i32p, c_int,
                                               c_float]),
            "orc_rope_tables": (None, [_f32p, _f32p, c_int, c_int, c_float]),
            "orc_rope_freqs": (None, [np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS"), c_int, c_float]),
            "orc_rope_freqs_llama3": (None, [np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS"), c_int,
                                             c_float, c_float, c_float, c_float, c_int]),
            "orc_rope_tables_llama3": (None, [_f32p, _f32p, c_int, c_int, c_float, c_float, c_float, c_float,
                                              c_int]),
            "orc_sigmoid": (c_float, [c_float]),
            "orc_swiglu": (None, [_f32p, _f32p, _f32p, c_ll]),
            "orc_quantize_rows": (None, [_i8p, _f32p, _f32p, c_int, c_int, c_int]),
            "orc_swiglu_q8_rows": (None, [_i8p, _f32p, _f32p, _f32p, c_int, c_int, c_int]),
            "orc_embedding_gather": (None, [_f32p, _i32p, c_int, c_int, _i8p, _f32p]),
            "orc_rmsnorm_rows": (None, [_f32p, _f32p, _f32p, c_int, c_int, c_float]),
            "orc_rmsnorm_quantize_rows": (None, [_i8p, _f32p, _f32p, _f32p, c_int, c_int, c_int, c_float]),
            "orc_add_inplace": (None, [_f32p, _f32p, c_ll]),
            "orc_kv_pack_f16": (None, [_u16p, _f32p, c_ll]),
            "orc_rope_only_heads": (None, [_f32p, c_int, c_int, _f32p, _f32p, c_int, c_int]),
            "orc_avx2_rope_only_heads": (None, [_f32p, c_int, c_int, _f32p, _f32p, c_int, c_int]),
            "orc_bias_add": (None, [_f32p, _f32p, c_ll]),
            "orc_avx2_kv_pack_f16": (None, [_u16p, _f32p, c_ll]),
            "orc_f16c_available": (c_int, []),
            "orc_check_f16_vs_f16c": (ctypes.c_ulonglong, [ctypes.c_uint64, ctypes.c_uint64, c_int]),
            "orc_avx2_available": (c_int, []),
            "orc_avx2_fused_add_rmsnorm": (None, [_f32p, _f32p, _f32p, _f32p, c_int, c_float]),
            "orc_avx2_rmsnorm_rope_heads": (None, [_f32p, c_int, c_int, _f32p, _f32p, _f32p, c_int, c_int, c_float]),
            "orc_avx2_swiglu": (None, [_f32p, _f32p, _f32p, c_ll]),
            "orc_avx2_quantize": (None, [_i8p, _f32p, _f32p, c_ll, c_int]),
            "orc_avx2_embedding_row": (None, [_f32p, c_int, c_int, _i8p, _f32p]),
            "orc_set_reference_fp_env": (None, [c_int]),
            "orc_get_reference_fp_env": (c_int, []),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


class gradual_underflow:
    """Context manager: the oracle's path functions run with IEEE gradual underflow instead of the
    reference's MXCSR FTZ+DAZ (v7_oracle.h), to show what that mode changes."""

    def __enter__(self):
        self._old = lib().orc_get_reference_fp_env()
        lib().orc_set_reference_fp_env(0)
        return self

    def __exit__(self, *exc):
        lib().orc_set_reference_fp_env(self._old)
        return False


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


# --------------------------------------------------------------------------- lane-faithful oracle

def fused_add_rmsnorm(residual, add, weight, eps):
    """Returns (o, residual_updated) for rows x dim inputs (copies; inputs untouched)."""
    r = _c(residual, np.float32).copy()
    a = _c(add, np.float32)
    w = _c(weight, np.float32)
    rows, dim = r.reshape(-1, r.shape[-1]).shape
    o = np.empty_like(r)
    lib().orc_fused_add_rmsnorm_rows(o, r, a, w, rows, dim, eps)
    return o, r


def sumsq_lanes(x):
    x = _c(x, np.float32)
    return np.float32(lib().orc_sumsq_lanes(x, x.size))


def rms_scale(ss, n, eps):
    return np.float32(lib().orc_rms_scale(float(ss), int(n), float(eps)))


def rmsnorm_rope(buf, norm_weight, cos_table, sin_table, positions, eps):
    """buf [T, H, D] -> new array; positions [T] int32; tables [P, rope_max_dim]."""
    b = _c(buf, np.float32).copy()
    T, H, D = b.shape
    ct = _c(cos_table, np.float32)
    st = _c(sin_table, np.float32)
    pos = _c(positions, np.int32)
    lib().orc_rmsnorm_rope_tokens(b, T, H * D, H, D, _c(norm_weight, np.float32), ct, st, pos, ct.shape[-1], eps)
    return b


def rope_tables(n_pos, head_dim, base):
    half = head_dim // 2
    c = np.empty((n_pos, half), np.float32)
    s = np.empty((n_pos, half), np.float32)
    lib().orc_rope_tables(c, s, n_pos, head_dim, float(base))
    return c, s


def rope_freqs(half, base):
    f = np.empty(half, np.float64)
    lib().orc_rope_freqs(f, half, float(base))
    return f


def rope_freqs_llama3(half, base, factor, low_freq_factor, high_freq_factor, orig_max_pos):
    """Llama 3 scaled RoPE frequencies (double), src/asm/fused_f32_kernel.inc:149-256."""
    f = np.empty(half, np.float64)
    lib().orc_rope_freqs_llama3(f, half, base, factor, low_freq_factor, high_freq_factor, orig_max_pos)
    return f


def rope_tables_llama3(n_pos, head_dim, base, factor, low_freq_factor, high_freq_factor, orig_max_pos):
    half = head_dim // 2
    c = np.empty((n_pos, half), np.float32)
    s = np.empty((n_pos, half), np.float32)
    lib().orc_rope_tables_llama3(c, s, n_pos, head_dim, base, factor, low_freq_factor, high_freq_factor, orig_max_pos)
    return c, s


def sigmoid(g):
    return np.float32(lib().orc_sigmoid(float(g)))


def swiglu(gate, up):
    g = _c(gate, np.float32)
    u = _c(up, np.float32)
    out = np.empty_like(g)
    lib().orc_swiglu(out, g, u, g.size)
    return out


def quantize(x, gs, row_len=None):
    """x [rows, row_len] (or flat with row_len) -> (codes int8 same shape, scales [rows, ceil(row_len/gs)])."""
    x = _c(x, np.float32)
    if row_len is None:
        row_len = x.shape[-1]
    rows = x.size // row_len
    spr = -(-row_len // gs)
    q = np.empty(x.size, np.int8)
    s = np.empty(rows * spr, np.float32)
    lib().orc_quantize_rows(q, x.reshape(-1), s, rows, row_len, gs)
    return q.reshape(x.shape), s.reshape(rows, spr)


def swiglu_q8(gate, up, gs):
    g = _c(gate, np.float32)
    u = _c(up, np.float32)
    hidden = g.shape[-1]
    rows = g.size // hidden
    spr = -(-hidden // gs)
    q = np.empty(g.size, np.int8)
    s = np.empty(rows * spr, np.float32)
    lib().orc_swiglu_q8_rows(q, s, g.reshape(-1), u.reshape(-1), rows, hidden, gs)
    return q.reshape(g.shape), s.reshape(rows, spr)


def embedding_gather(ids, table_q, table_s, dim):
    ids = _c(ids, np.int32)
    out = np.empty((ids.size, dim), np.float32)
    lib().orc_embedding_gather(out, ids, ids.size, dim, _c(table_q, np.int8).reshape(-1),
                               _c(table_s, np.float32).reshape(-1))
    return out


def rmsnorm(x, weight, eps):
    """v7s_rmsnorm per row of x [rows, dim]."""
    x = _c(x, np.float32)
    dim = x.shape[-1]
    o = np.empty_like(x)
    lib().orc_rmsnorm_rows(o, x, _c(weight, np.float32), x.size // dim, dim, eps)
    return o


def rmsnorm_quantize(x, weight, eps, gs=64):
    """v7s_rmsnorm_quantize per row: (codes like x, scales [rows, ceil(dim/gs)])."""
    x = _c(x, np.float32)
    dim = x.shape[-1]
    rows = x.size // dim
    spr = -(-dim // gs)
    q = np.empty(x.size, np.int8)
    s = np.empty(rows * spr, np.float32)
    lib().orc_rmsnorm_quantize_rows(q, s, x.reshape(-1), _c(weight, np.float32), rows, dim, gs, eps)
    return q.reshape(x.shape), s.reshape(rows, spr)


def rope_only(buf, cos_table, sin_table, positions):
    """v7s_rope_only_heads per token: buf [T, H, D] -> new array."""
    b = _c(buf, np.float32).copy()
    T, H, D = b.shape
    ct = _c(cos_table, np.float32)
    st = _c(sin_table, np.float32)
    for t in range(T):
        lib().orc_rope_only_heads(b[t].reshape(-1), H, D, ct, st, int(positions[t]), ct.shape[-1])
    return b


def bias_add(x, bias):
    """PQ_BIAS_ADD per token row: x [T, n] + bias [n] -> new array."""
    x = _c(x, np.float32).copy()
    b = _c(bias, np.float32).reshape(-1)
    for row in x.reshape(-1, b.size):
        lib().orc_bias_add(row, b, b.size)
    return x


def qkv_stage(q, k, v, q_w, k_w, q_bias, k_bias, v_bias, cos_table, sin_table, positions, eps):
    """Stage C of the Q8 prefill for T tokens (src/asm/prefill_q8.inc:848-883): per side, the bias add
    (if given), then RMSNorm+RoPE (norm weight given) or RoPE only, for Q and K; V gets the bias only.
    Returns (q, k, v, k_f16, v_f16) with the binary16 cache rows of K and V (v7s_kv_pack_f16)."""
    T = q.shape[0]
    qs, ks, vs = q.shape, k.shape, v.shape
    q2 = bias_add(q.reshape(T, -1), q_bias).reshape(qs) if q_bias is not None else _c(q, np.float32).copy()
    k2 = bias_add(k.reshape(T, -1), k_bias).reshape(ks) if k_bias is not None else _c(k, np.float32).copy()
    v2 = bias_add(v.reshape(T, -1), v_bias).reshape(vs) if v_bias is not None else _c(v, np.float32).copy()
    pos = np.asarray(positions, np.int32)
    q2 = rmsnorm_rope(q2, q_w, cos_table, sin_table, pos, eps) if q_w is not None else rope_only(q2, cos_table,
                                                                                                    sin_table, pos)
    k2 = rmsnorm_rope(k2, k_w, cos_table, sin_table, pos, eps) if k_w is not None else rope_only(k2, cos_table,
                                                                                                    sin_table, pos)
    return q2, k2, v2, kv_pack_f16(k2), kv_pack_f16(v2)


def kv_pack_f16(x):
    """v7s_kv_pack_f16: binary16 bit patterns (uint16, same shape) of x, round to nearest even."""
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_kv_pack_f16(out.reshape(-1), x.reshape(-1), x.size)
    return out


def f16c_available():
    return bool(lib().orc_f16c_available())


def avx2_kv_pack_f16(x):
    x = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_avx2_kv_pack_f16(out.reshape(-1), x.reshape(-1), x.size)
    return out


def check_f16_vs_f16c(lo, count, threads):
    return int(lib().orc_check_f16_vs_f16c(lo, count, threads))


def add_inplace(x, y):
    """v7s_add_inplace: returns x + y (a copy of x updated)."""
    x = _c(x, np.float32).copy()
    lib().orc_add_inplace(x.reshape(-1), _c(y, np.float32).reshape(-1), x.size)
    return x


# --------------------------------------------------------------------------- AVX2 restatement (CPU baseline)

def avx2_available():
    return bool(lib().orc_avx2_available())


def avx2_fused_add_rmsnorm_rows(residual, add, weight, eps):
    r = _c(residual, np.float32).copy()
    a = _c(add, np.float32)
    w = _c(weight, np.float32)
    o = np.empty_like(r)
    dim = r.shape[-1]
    for i in range(r.size // dim):
        ro, ao, oo = r.reshape(-1, dim)[i], a.reshape(-1, dim)[i], o.reshape(-1, dim)[i]
        lib().orc_avx2_fused_add_rmsnorm(oo, ro, ao, w, dim, eps)
    return o, r


def avx2_rmsnorm_rope(buf, norm_weight, cos_table, sin_table, positions, eps):
    b = _c(buf, np.float32).copy()
    T, H, D = b.shape
    ct = _c(cos_table, np.float32)
    st = _c(sin_table, np.float32)
    w = _c(norm_weight, np.float32)
    for t in range(T):
        lib().orc_avx2_rmsnorm_rope_heads(b[t], H, D, w, ct, st, int(positions[t]), ct.shape[-1], eps)
    return b


def avx2_swiglu(gate, up):
    g = _c(gate, np.float32)
    u = _c(up, np.float32)
    out = np.empty_like(g)
    lib().orc_avx2_swiglu(out, g, u, g.size)
    return out


def avx2_quantize(x, gs):
    x = _c(x, np.float32)
    row_len = x.shape[-1]
    rows = x.size // row_len
    spr = -(-row_len // gs)
    q = np.empty((rows, row_len), np.int8)
    s = np.empty((rows, spr), np.float32)
    xr = x.reshape(rows, row_len)
    for r in range(rows):
        lib().orc_avx2_quantize(q[r], xr[r], s[r], row_len, gs)
    return q.reshape(x.shape), s


def avx2_embedding_gather(ids, table_q, table_s, dim):
    ids = _c(ids, np.int32)
    out = np.empty((ids.size, dim), np.float32)
    tq = _c(table_q, np.int8).reshape(-1)
    ts = _c(table_s, np.float32).reshape(-1)
    for t in range(ids.size):
        lib().orc_avx2_embedding_row(out[t], int(ids[t]), dim, tq, ts)
    return out


# --------------------------------------------------------------------------- reference C checkers, restated

def kt_quantize_c_ref(x):
    """tools/kt_utils.h:378-407 (GS 64, float arithmetic, lrintf, all-zero scale 1/127)."""
    x = _c(x, np.float32).reshape(-1)
    n = x.size
    gs = 64
    ng = -(-n // gs)
    q = np.empty(n, np.int8)
    s = np.empty(ng, np.float32)
    for g in range(ng):
        seg = x[g * gs:(g + 1) * gs]
        wmax = np.float32(np.max(np.abs(seg))) if seg.size else np.float32(0)
        scale = np.float32(1.0) / np.float32(127.0) if wmax == 0 else wmax / np.float32(127.0)
        s[g] = scale
        recip = np.float32(1.0) / np.float32(scale)
        val = seg * recip
        qi = np.rint(val).astype(np.int64)
        q[g * gs:g * gs + seg.size] = np.clip(qi, -127, 127).astype(np.int8)
    return q, s


def kt_rmsnorm_c_ref(x, weight, eps):
    """tools/kt_utils.h:450-458, float accumulation in element order, o = x*scale*w."""
    x = _c(x, np.float32)
    ss = np.float32(0)
    for v in x:
        ss = np.float32(ss + np.float32(v * v))
    scale = np.float32(1.0) / np.sqrt(np.float32(ss / np.float32(x.size) + np.float32(eps)))
    return ((x * scale).astype(np.float32) * _c(weight, np.float32)).astype(np.float32)


def kt_fused_add_rmsnorm_c_ref(residual, add, weight, eps):
    """tools/kt_utils.h:493-503, float accumulation in element order."""
    r = (_c(residual, np.float32) + _c(add, np.float32)).astype(np.float32)
    ss = np.float32(0)
    for v in r:
        ss = np.float32(ss + np.float32(v * v))
    scale = np.float32(1.0) / np.sqrt(np.float32(ss / np.float32(r.size) + np.float32(eps)))
    return (r * scale * _c(weight, np.float32)).astype(np.float32), r


def rmsnorm_rope_double_ref(buf, norm_weight, cos_table, sin_table, positions, eps):
    """tools/kt_utils.h:460-485 vectorised: double sum of squares and rotation, per head."""
    b = np.asarray(buf, np.float64)
    T, H, D = b.shape
    half = D // 2
    ss = np.sum(b * b, axis=-1, keepdims=True)
    scale = 1.0 / np.sqrt(ss / D + float(eps))
    qn = (b * np.asarray(norm_weight, np.float64) * scale).astype(np.float32).astype(np.float64)
    pos = np.asarray(positions)
    c = np.asarray(cos_table, np.float64)[pos][:, None, :half]
    s = np.asarray(sin_table, np.float64)[pos][:, None, :half]
    x0, y0 = qn[..., :half], qn[..., half:]
    out = np.empty_like(qn)
    out[..., :half] = x0 * c - y0 * s
    out[..., half:] = x0 * s + y0 * c
    return out.astype(np.float32)
