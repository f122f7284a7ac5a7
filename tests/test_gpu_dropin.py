"""GPU parity of the drop-in entries (reference names and ms_abi calling convention), one row per call.

Each entry is called through tests/libdropin_shim.so, whose System V wrappers make the ms_abi call the
way a v7 host would (src/v7_lib.h:40-46,123,272-275).  Outputs must equal the oracle bit for bit;
eps comes from the library global, as the reference's g_rms_eps (src/asm/v7_data.inc:509).
"""
from __future__ import annotations

import ctypes
import os

import numpy as np
import pytest

from tests import common as C

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

SHIM = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libdropin_shim.so")


@pytest.fixture(scope="module")
def shim():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a visible MI355X")
    from v7multiplikator_amd import _lib
    L = _lib.load()
    if not os.path.exists(SHIM):
        pytest.fail(f"{SHIM} is missing: run __graft_entry__.build()")
    S = ctypes.CDLL(SHIM)
    vp, i, f = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
    S.shim_fused_add_rmsnorm.argtypes = [vp, vp, vp, vp, i]
    S.shim_rmsnorm_rope_heads.argtypes = [vp, i, i, vp, vp, vp, i, i]
    S.shim_quantize.argtypes = [vp, vp, vp, i]
    S.shim_embedding_row.argtypes = [vp, i, i, vp, vp]
    S.shim_swiglu_row.argtypes = [vp, vp, i]
    S.shim_swiglu_quantize_row.argtypes = [vp, vp, vp, vp, i]
    S.shim_rope_init.argtypes = [i, f]
    S.shim_rmsnorm.argtypes = [vp, vp, vp, i]
    S.shim_rmsnorm_quantize.argtypes = [vp, vp, vp, i, vp]
    S.shim_add_inplace.argtypes = [vp, vp, i]
    S.shim_kv_pack_f16.argtypes = [vp, vp, i]
    S.shim_rope_only_heads.argtypes = [vp, i, i, vp, vp, i, i]
    S.shim_qk_fork_heads.argtypes = [vp, vp, vp, vp, i, i, i]
    torch.cuda.synchronize()
    L.v7g_set_stream(torch.cuda.current_stream().cuda_stream)
    L.v7g_clear_last_error()
    yield S, L
    L.v7g_set_rms_eps(1e-6)


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def done(L):
    assert L.v7g_sync() == 0
    err = L.v7g_get_last_error()
    L.v7g_clear_last_error()
    assert err == 0, err


def bits(a, b):
    a, b = np.asarray(a), np.asarray(b)
    if a.dtype.kind == "f":
        return np.array_equal(a.view(np.uint32), b.view(np.uint32))
    return np.array_equal(a, b)


@pytest.mark.parametrize("dim", [8, 24, 40, 2048, 4096])
@pytest.mark.parametrize("eps", [1e-6, 1e-5])
def test_v7s_fused_add_rmsnorm_rows(shim, oracle, dim, eps):
    S, L = shim
    L.v7g_set_rms_eps(eps)
    rows = 3
    r = C.validator_row(dim, rows * dim).reshape(rows, dim)
    a = C.validator_row(dim + 1, rows * dim).reshape(rows, dim)
    w = C.validator_weight(dim + 2, dim)
    rt, at, wt = dev(r), dev(a), dev(w)
    ot = torch.empty_like(rt)
    for k in range(rows):  # one call per row, as forward_f32.inc:324-332 calls it
        S.shim_fused_add_rmsnorm(ot[k].data_ptr(), rt[k].data_ptr(), at[k].data_ptr(), wt.data_ptr(), dim)
    done(L)
    want_o, want_r = oracle.fused_add_rmsnorm(r, a, w, eps)
    assert bits(rt.cpu().numpy(), want_r) and bits(ot.cpu().numpy(), want_o)


@pytest.mark.parametrize("heads,hd,pos", [(1, 64, 0), (4, 64, 7), (16, 128, 31), (8, 96, 5), (40, 128, 1000)])
def test_v7s_rmsnorm_rope_heads_per_token(shim, oracle, heads, hd, pos):
    S, L = shim
    L.v7g_set_rms_eps(1e-6)
    buf = C.normal(heads + hd, (1, heads, hd))
    w = C.norm_weight(hd, hd)
    ct, st = oracle.rope_tables(pos + 1, hd, 1e6)
    bt, wt, ctt, stt = dev(buf), dev(w), dev(ct), dev(st)
    S.shim_rmsnorm_rope_heads(bt.data_ptr(), heads, hd, wt.data_ptr(), ctt.data_ptr(), stt.data_ptr(), pos, hd // 2)
    done(L)
    want = oracle.rmsnorm_rope(buf, w, ct, st, np.array([pos], np.int32), 1e-6)
    assert bits(bt.cpu().numpy(), want)


@pytest.mark.parametrize("n", [64, 100, 4096, 8192 + 17])
def test_v7d_quantize(shim, oracle, n):
    S, L = shim
    x = C.normal(n, n, 2.0)
    xt = dev(x)
    qt = torch.empty(n, dtype=torch.int8, device="cuda")
    st = torch.empty(-(-n // 64), dtype=torch.float32, device="cuda")
    S.shim_quantize(qt.data_ptr(), xt.data_ptr(), st.data_ptr(), n)
    done(L)
    wq, ws = oracle.quantize(x[None], 64)
    assert bits(qt.cpu().numpy(), wq[0]) and bits(st.cpu().numpy(), ws[0])


@pytest.mark.parametrize("dim", [64, 256, 896, 4096])
def test_v7s_embedding_row(shim, oracle, dim):
    """One row per call (no id array: the table is offset to the row): the one-workgroup-per-row kernel below
    256 codes, the flat-piece kernel's last group of workgroups (its bounds-tested path) from 256 on."""
    S, L = shim
    vocab = 300
    tq, ts = C.q8_table(31, vocab, dim)
    tqt, tst = dev(tq), dev(ts)
    ids = [0, 7, 299, 150]
    out = torch.empty((len(ids), dim), dtype=torch.float32, device="cuda")
    for k, t in enumerate(ids):  # one call per token, as prefill_q8.inc:317-350 calls it
        S.shim_embedding_row(out[k].data_ptr(), t, dim, tqt.data_ptr(), tst.data_ptr())
    done(L)
    assert bits(out.cpu().numpy(), oracle.embedding_gather(np.array(ids, np.int32), tq, ts, dim))


@pytest.mark.parametrize("hidden", [64, 1000, 12288])
def test_v7s_swiglu_row_in_place_and_quantize_row(shim, oracle, hidden):
    S, L = shim
    g = C.normal(hidden, hidden, 1.5)
    u = C.normal(hidden + 1, hidden, 1.5)
    gt, ut = dev(g), dev(u)
    S.shim_swiglu_row(gt.data_ptr(), ut.data_ptr(), hidden)  # in place over the gate row, as .pq_ffn_silu
    done(L)
    assert bits(gt.cpu().numpy(), oracle.swiglu(g, u))
    gt2 = dev(g)
    qt = torch.empty(hidden, dtype=torch.int8, device="cuda")
    st = torch.empty(-(-hidden // 64), dtype=torch.float32, device="cuda")
    S.shim_swiglu_quantize_row(qt.data_ptr(), gt2.data_ptr(), ut.data_ptr(), st.data_ptr(), hidden)
    done(L)
    wq, ws = oracle.swiglu_q8(g[None], u[None], 64)  # hidden 1000: a 40-element tail group
    assert bits(qt.cpu().numpy(), wq[0]) and bits(st.cpu().numpy(), ws[0])
    assert bits(gt2.cpu().numpy(), g)  # gate untouched by the fused form


def test_v7s_rope_init_tables(shim, oracle):
    S, L = shim
    S.shim_rope_init(128, ctypes.c_float(1e6))
    done(L)
    c = ctypes.c_void_p()
    s = ctypes.c_void_p()
    rmd = ctypes.c_int()
    npos = ctypes.c_int()
    assert L.v7g_get_rope_tables(ctypes.byref(c), ctypes.byref(s), ctypes.byref(rmd), ctypes.byref(npos)) == 0
    assert rmd.value == 64 and npos.value == 131072
    # the first 4096 rows, copied from the library-owned device tables into torch tensors
    n = 4096 * 64
    tc = torch.empty(n, dtype=torch.float32, device="cuda")
    ts_ = torch.empty(n, dtype=torch.float32, device="cuda")
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    assert hip.hipMemcpy(tc.data_ptr(), c.value, n * 4, 3) == 0  # hipMemcpyDeviceToDevice
    assert hip.hipMemcpy(ts_.data_ptr(), s.value, n * 4, 3) == 0
    wc, ws = oracle.rope_tables(4096, 128, 1e6)
    assert bits(tc.cpu().numpy(), wc.reshape(-1)) and bits(ts_.cpu().numpy(), ws.reshape(-1))


def _owned_tables(L, rows, half):
    c, s, rmd, npos = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_int(), ctypes.c_int()
    assert L.v7g_get_rope_tables(ctypes.byref(c), ctypes.byref(s), ctypes.byref(rmd), ctypes.byref(npos)) == 0
    assert rmd.value == half and npos.value == 131072
    tc = torch.empty(rows * half, dtype=torch.float32, device="cuda")
    ts_ = torch.empty(rows * half, dtype=torch.float32, device="cuda")
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    assert hip.hipMemcpy(tc.data_ptr(), c.value, tc.numel() * 4, 3) == 0  # hipMemcpyDeviceToDevice
    assert hip.hipMemcpy(ts_.data_ptr(), s.value, ts_.numel() * 4, 3) == 0
    return tc.cpu().numpy().reshape(rows, half), ts_.cpu().numpy().reshape(rows, half)


def test_v7s_rope_init_follows_the_model_config(shim, oracle):
    """With the model's RoPE configuration set (the stand-in for the DB keys the reference's builder reads,
    src/asm/fused_f32_kernel.inc:97-110,149-256), an unchanged v7s_rope_init(head_dim, 0.0f) builds the Llama 3
    scaled tables; a type-0 configuration makes it ignore its float argument; cleared, the argument counts again."""
    S, L = shim
    f = ctypes.c_float
    try:
        assert L.v7g_set_rope_config(1, f(500000.0), f(8.0), f(1.0), f(4.0), 8192) == 0
        S.shim_rope_init(128, f(0.0))
        done(L)
        wc, ws = oracle.rope_tables_llama3(2048, 128, 500000.0, 8.0, 1.0, 4.0, 8192)
        gc, gs = _owned_tables(L, 2048, 64)
        assert bits(gc, wc) and bits(gs, ws)
        assert L.v7g_set_rope_config(0, f(1e4), f(0.0), f(0.0), f(0.0), 0) == 0
        S.shim_rope_init(64, f(1e6))  # the argument is ignored: the configured base is 1e4
        done(L)
        wc, ws = oracle.rope_tables(1024, 64, 1e4)
        gc, gs = _owned_tables(L, 1024, 32)
        assert bits(gc, wc) and bits(gs, ws)
        L.v7g_clear_rope_config()
        S.shim_rope_init(64, f(1e6))
        done(L)
        wc, ws = oracle.rope_tables(1024, 64, 1e6)
        gc, gs = _owned_tables(L, 1024, 32)
        assert bits(gc, wc) and bits(gs, ws)
    finally:
        L.v7g_clear_rope_config()


@pytest.mark.parametrize("size", [64, 1024, 3072, 8192])
def test_v7s_rmsnorm_and_rmsnorm_quantize(shim, oracle, size):
    S, L = shim
    L.v7g_set_rms_eps(1e-5)
    x = C.validator_row(size, size)
    w = C.validator_weight(size + 1, size)
    xt, wt = dev(x), dev(w)
    ot = torch.empty_like(xt)
    S.shim_rmsnorm(ot.data_ptr(), xt.data_ptr(), wt.data_ptr(), size)
    qt = torch.empty(size, dtype=torch.int8, device="cuda")
    st = torch.empty(size // 64, dtype=torch.float32, device="cuda")
    S.shim_rmsnorm_quantize(qt.data_ptr(), xt.data_ptr(), st.data_ptr(), size, wt.data_ptr())
    done(L)
    assert bits(ot.cpu().numpy(), oracle.rmsnorm(x[None], w, 1e-5)[0])
    wq, ws = oracle.rmsnorm_quantize(x[None], w, 1e-5, 64)
    assert bits(qt.cpu().numpy(), wq[0]) and bits(st.cpu().numpy(), ws[0])


@pytest.mark.parametrize("n", [32, 64, 96, 128, 160, 1024, 2048, 2051])  # tools/v_add_inplace_validate.cpp's sizes
def test_v7s_add_inplace(shim, oracle, n):
    S, L = shim
    x = C.validator_row(n, n)
    y = C.validator_row(n + 1, n)
    xt, yt = dev(x), dev(y)
    S.shim_add_inplace(xt.data_ptr(), yt.data_ptr(), n)
    done(L)
    assert bits(xt.cpu().numpy(), oracle.add_inplace(x, y))


@pytest.mark.parametrize("count", [8, 24, 1024, 8 * 128])
def test_v7s_kv_pack_f16_row(shim, oracle, count):
    S, L = shim
    x = C.normal(count, count, 4.0)
    xt = dev(x)
    ht = torch.empty(count, dtype=torch.float16, device="cuda")
    S.shim_kv_pack_f16(ht.data_ptr(), xt.data_ptr(), count)
    done(L)
    assert bits(ht.cpu().numpy().view(np.uint16), oracle.kv_pack_f16(x))


@pytest.mark.parametrize("heads,hd,pos", [(1, 64, 0), (4, 64, 7), (16, 128, 31), (8, 96, 5), (8, 128, 4000)])
def test_v7s_rope_only_heads_per_token(shim, oracle, heads, hd, pos):
    S, L = shim
    buf = C.normal(heads * hd + pos, (1, heads, hd))
    ct, st = oracle.rope_tables(pos + 1, hd, 1e4)
    bt, ctt, stt = dev(buf), dev(ct), dev(st)
    S.shim_rope_only_heads(bt.data_ptr(), heads, hd, ctt.data_ptr(), stt.data_ptr(), pos, hd // 2)
    done(L)
    assert bits(bt.cpu().numpy(), oracle.rope_only(buf, ct, st, np.array([pos], np.int32)))


@pytest.mark.parametrize("heads,hd,pos,rmd", [(8, 128, 0, 64), (32, 128, 17, 64), (8, 128, 300, 96), (4, 64, 5, 32),
                                              (2, 256, 9, 128)])
def test_v7s_qk_fork_heads_descriptor(shim, oracle, heads, hd, pos, rmd):
    """The descriptor form (src/asm/qk_fork_kernel.inc:10-62): cos/sin pre-offset to row pos of a table with
    rope_max_dim floats per row (rmd >= head_dim/2), exactly what v7s_rmsnorm_rope_heads computes."""
    S, L = shim
    L.v7g_set_rms_eps(1e-6)
    buf = C.normal(heads * hd + pos, (1, heads, hd))
    w = C.norm_weight(hd + 1, hd)
    c0, s0 = oracle.rope_tables(pos + 1, hd, 1e6)
    ct = np.full((pos + 1, rmd), np.nan, np.float32)  # a wider table: the columns past head_dim/2 are never read
    st = np.full((pos + 1, rmd), np.nan, np.float32)
    ct[:, : hd // 2], st[:, : hd // 2] = c0, s0
    bt, wt, ctt, stt = dev(buf), dev(w), dev(ct), dev(st)
    row = pos * rmd * 4
    S.shim_qk_fork_heads(bt.data_ptr(), wt.data_ptr(), ctt.data_ptr() + row, stt.data_ptr() + row, hd, heads, pos)
    done(L)
    want = oracle.rmsnorm_rope(buf, w, ct, st, np.array([pos], np.int32), 1e-6)
    assert bits(bt.cpu().numpy(), want)
