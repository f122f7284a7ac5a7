"""Overlapping outputs are refused at the C ABI before any launch (CPU only).

Every kernel reads and writes in one pass with many workgroups in flight, so an
output that shares bytes with another argument would race.  The reference's
prefill quantizes the SwiGLU row into the retired up row
(src/asm/prefill_q8.inc:1169-1180), safe there because its SwiGLU pass ends
before the quantizer starts; ported onto the fused SwiGLU -> Q8 entry that
layout must be rejected.  The entries accept only the exact in-place forms
their declarations list (include/v7g_lib.h).

The overlap arithmetic itself (csrc/v7g_alias.h) is checked against a
byte-by-byte intersection by tests/alias_check.cpp.  The rejection tests use
fabricated addresses: an entry that failed to refuse would try to launch, so
they run only where no GPU is present.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
import tempfile

import pytest

from v7multiplikator_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ALIAS = _lib.V7G_ERR_ALIAS
BASE = 0x7F0000000000  # fabricated, 256-byte aligned; never dereferenced

no_gpu = pytest.mark.skipif("__import__('torch').cuda.is_available()",
                            reason="a missed refusal would launch on fabricated addresses")


def test_span_overlap_matches_brute_force():
    with tempfile.TemporaryDirectory() as d:
        exe = os.path.join(d, "alias_check")
        subprocess.run(["g++", "-O2", "-std=c++17", "-o", exe, os.path.join(ROOT, "tests", "alias_check.cpp")],
                       check=True)
        r = subprocess.run([exe, "300000"], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout
    pairs, hits = (int(x) for x in r.stdout.split()[1:4:2])
    assert pairs == 300000 and 0.2 * pairs < hits < 0.9 * pairs  # both outcomes well represented


@pytest.fixture(scope="module")
def L():
    return _lib.load()


def _rc(L, fn, *args):
    L.v7g_clear_last_error()
    rc = fn(*args)
    assert L.v7g_get_last_error() == rc
    return rc


def test_error_string(L):
    assert L.v7g_error_string(ALIAS) == b"an output overlaps another argument"


@no_gpu
def test_swiglu_q8_codes_over_the_retired_up_row(L):
    """The reference's layout (codes at up, scales at up + hidden bytes) and its variants are refused."""
    rows, hidden, gs = 4, 256, 64
    gate, up = BASE, BASE + rows * hidden * 4
    assert _rc(L, L.v7g_swiglu_q8, up, up + hidden, gate, up, 1, hidden, 64) == ALIAS
    assert _rc(L, L.v7g_swiglu_q8, up, up + rows * hidden * 4, gate, up, rows, hidden, gs) == ALIAS
    assert _rc(L, L.v7g_swiglu_q8, gate + 1024, BASE + (1 << 24), gate, up, rows, hidden, gs) == ALIAS  # codes in gate
    assert _rc(L, L.v7g_swiglu_q8, BASE + (1 << 24), up + 4 * (rows * hidden - 1), gate, up, rows, hidden,
               gs) == ALIAS  # a scale on up's last float
    codes = BASE + (1 << 24)
    assert _rc(L, L.v7g_swiglu_q8, codes, codes + rows * hidden - 4, gate, up, rows, hidden, gs) == ALIAS  # codes/scales
    assert _rc(L, L.v7g_quantize_q8, gate, codes, gate, rows, hidden, gs) == ALIAS  # in place over x


@no_gpu
def test_norm_quantize_outputs_apart(L):
    rows, dim, gs = 4, 256, 64
    x, w, q, s = BASE, BASE + (1 << 20), BASE + (2 << 20), BASE + (3 << 20)
    assert _rc(L, L.v7g_rmsnorm_quantize, x, s, x, w, rows, dim, gs, ctypes.c_float(1e-6)) == ALIAS
    assert _rc(L, L.v7g_rmsnorm_quantize, q, x + 16, x, w, rows, dim, gs, ctypes.c_float(1e-6)) == ALIAS
    assert _rc(L, L.v7g_rmsnorm_quantize, q, s, x, q + 64, rows, dim, gs, ctypes.c_float(1e-6)) == ALIAS  # weight
    assert _rc(L, L.v7g_rmsnorm_quantize, q, q + 512, x, w, rows, dim, gs, ctypes.c_float(1e-6)) == ALIAS  # q/s
    a = BASE + (4 << 20)
    assert _rc(L, L.v7g_add_rmsnorm_quantize, q, s, x, x, w, rows, dim, gs, ctypes.c_float(1e-6)) == ALIAS  # add = residual
    assert _rc(L, L.v7g_add_rmsnorm_quantize, a, s, x, a, w, rows, dim, gs, ctypes.c_float(1e-6)) == ALIAS  # codes in add
    assert _rc(L, L.v7g_add_rmsnorm_quantize, q, s, x, a, x + 4080, rows, dim, gs, ctypes.c_float(1e-6)) == ALIAS


@no_gpu
def test_norms_accept_only_exact_in_place(L):
    rows, dim = 4, 256
    o, r, a, w = BASE, BASE + (1 << 20), BASE + (2 << 20), BASE + (3 << 20)
    eps = ctypes.c_float(1e-6)
    assert _rc(L, L.v7g_fused_add_rmsnorm, r + 16, r, a, w, rows, dim, eps) == ALIAS  # shifted in-place
    assert _rc(L, L.v7g_fused_add_rmsnorm, a + 1024, r, a, w, rows, dim, eps) == ALIAS  # o one row into add
    assert _rc(L, L.v7g_fused_add_rmsnorm, o, r, r, w, rows, dim, eps) == ALIAS  # add = residual
    assert _rc(L, L.v7g_fused_add_rmsnorm, o, r, a, o + 64, rows, dim, eps) == ALIAS  # weight inside o
    assert _rc(L, L.v7g_fused_add_rmsnorm, o, r, a, r + 4 * rows * dim - 16, rows, dim, eps) == ALIAS  # weight tail
    assert _rc(L, L.v7g_rmsnorm, r + 1024, r, w, rows, dim, eps) == ALIAS
    assert _rc(L, L.v7g_rmsnorm, o, r, o + 16, rows, dim, eps) == ALIAS
    assert _rc(L, L.v7g_add_inplace, r, r + 16, 1024) == ALIAS
    assert _rc(L, L.v7g_swiglu_f32, a + 16, a, r, 1024) == ALIAS
    assert _rc(L, L.v7g_swiglu_f32, r - 16, a, r, 1024) == ALIAS


@no_gpu
def test_rope_heads_and_caches_apart(L):
    T, HD, NQ, NK = 8, 128, 4, 2
    stride = (NQ + 2 * NK) * HD  # a fused QKV row, in floats
    qkv = BASE
    q, k, v = qkv, qkv + NQ * HD * 4, qkv + (NQ + NK) * HD * 4
    qw, kw = BASE + (1 << 20), BASE + (1 << 20) + 4096
    cos, sin = BASE + (2 << 20), BASE + (3 << 20)
    eps = ctypes.c_float(1e-6)
    # K starting inside Q's heads of the same token
    assert _rc(L, L.v7g_qk_rmsnorm_rope, q, stride, NQ, qw, q + 256, stride, NK, kw, T, HD, cos, sin, None, 0, 64, T,
               eps) == ALIAS
    # K one token row later than the QKV layout puts it: overlaps Q of the next token
    assert _rc(L, L.v7g_qk_rmsnorm_rope, q, stride, NQ, qw, q + stride * 4 - 256, stride, NK, kw, T, HD, cos, sin,
               None, 0, 64, T, eps) == ALIAS
    # heads over the table or the weights
    assert _rc(L, L.v7g_rmsnorm_rope_heads, cos + 1024, 1, 0, 1, HD, qw, cos, sin, None, 0, 64, T, eps) == ALIAS
    assert _rc(L, L.v7g_rmsnorm_rope_heads, qw - 256, 1, 0, 1, HD, qw, cos, sin, None, 0, 64, T, eps) == ALIAS
    assert _rc(L, L.v7g_rope_only_heads, sin, T, stride, NQ, HD, cos, sin, None, 0, 64, T) == ALIAS
    # binary16 K cache rows over the K heads' second half, same row stride
    kc = k + 512
    assert _rc(L, L.v7g_qk_rmsnorm_rope_kv, q, stride, NQ, qw, k, stride, NK, kw, T, HD, cos, sin, None, 0, 64, T,
               eps, kc, stride * 2, 1) == ALIAS
    st = _lib.QkvStage()
    st.q = _lib.QkvSide(q, stride, NQ, qw, None, None, 0, 1)
    st.k = _lib.QkvSide(k, stride, NK, kw, None, BASE + (4 << 20), NK * HD, 1)
    st.v = _lib.QkvSide(v, stride, NK, None, None, BASE + (4 << 20) + NK * HD * 2 - 8, NK * HD, 1)  # V rows over K's
    st.n_tokens, st.head_dim, st.cos_table, st.sin_table = T, HD, cos, sin
    st.positions, st.pos0, st.rope_max_dim, st.table_rows, st.eps = None, 0, 64, T, 1e-6
    assert _rc(L, L.v7g_qkv_rope_stage, ctypes.byref(st)) == ALIAS
    st.v = _lib.QkvSide(v, stride, NK, None, None, q + 64, NK * HD, 1)  # V cache inside Q's heads
    assert _rc(L, L.v7g_qkv_rope_stage, ctypes.byref(st)) == ALIAS
    st.v = _lib.QkvSide(v, stride, NK, None, BASE + (4 << 20) + 256, BASE + (8 << 20), NK * HD, 1)  # K cache over V bias
    assert _rc(L, L.v7g_qkv_rope_stage, ctypes.byref(st)) == ALIAS


@no_gpu
def test_kv_pack_embedding_and_tables_apart(L):
    rows, row_len = 8, 256
    src = BASE
    assert _rc(L, L.v7g_kv_pack_f16, src, row_len, src, row_len, rows, row_len) == ALIAS  # in place
    assert _rc(L, L.v7g_kv_pack_f16, src + rows * row_len * 4 - 8, row_len, src, row_len, rows, row_len) == ALIAS
    # dst rows interleaved with src rows of the same byte stride, sharing one byte range
    assert _rc(L, L.v7g_kv_pack_f16, src + row_len * 4 - 8, 2 * (2 * row_len), src, 2 * row_len, rows,
               row_len) == ALIAS
    # the one-launch K/V form: V cache over the K cache, K cache over the V source rows
    kc, vc = BASE + (4 << 20), BASE + (5 << 20)
    assert _rc(L, L.v7g_kv_pack_f16_kv, kc, row_len, kc + 512, row_len, src, src + row_len * 4, 3 * row_len, rows,
               row_len) == ALIAS
    assert _rc(L, L.v7g_kv_pack_f16_kv, src + row_len * 4 + 8, 6 * row_len, vc, row_len, src, src + row_len * 4,
               3 * row_len, rows, row_len) == ALIAS
    ids, tq, ts = BASE + (1 << 20), BASE + (2 << 20), BASE + (3 << 20)
    assert _rc(L, L.v7g_embedding_gather_q8, tq + 4096, ids, 4, tq, ts, 128, 100) == ALIAS
    assert _rc(L, L.v7g_embedding_gather_q8, ts, ids, 4, tq, ts, 128, 100) == ALIAS
    assert _rc(L, L.v7g_embedding_gather_q8, ids - 16, ids, 4, tq, ts, 128, 100) == ALIAS
    f = ctypes.c_float
    assert _rc(L, L.v7g_build_rope_tables, BASE, BASE + 16 * 64 * 4 - 4, 16, 128, f(1e6)) == ALIAS
    assert _rc(L, L.v7g_build_rope_tables_llama3, BASE, BASE, 16, 128, f(5e5), f(8), f(1), f(4), 8192) == ALIAS


@no_gpu
def test_refusal_comes_before_any_launch_and_is_sticky(L):
    """The sticky error keeps ALIAS; the call made no HIP launch (a launch here, without a device, would have
    recorded V7G_ERR_HIP instead)."""
    L.v7g_clear_last_error()
    assert L.v7g_swiglu_q8(BASE, BASE + 64, BASE, BASE + 4096, 1, 256, 64) == ALIAS
    assert L.v7g_get_last_error() == ALIAS
    L.v7g_clear_last_error()
