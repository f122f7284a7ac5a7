"""GPU: the layouts the overlap rule allows, and a refused call, through the C ABI.

The reference's prefill puts the SwiGLU row's Q8 codes and scales into the
retired up row (src/asm/prefill_q8.inc:1169-1180).  Here codes and scales need
their own memory, and the natural replacement keeps them in the same arena,
right after up: that layout must stay bit-exact.  The exact in-place forms the
entries accept (add+RMSNorm's o equal to residual or add, SwiGLU's out equal to
gate or up, add_inplace's y equal to x) must equal the out-of-place results; an
overlapping call must be refused without touching memory.
"""
from __future__ import annotations

import numpy as np
import pytest

from tests import common as C

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module")
def L():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a visible MI355X")
    from v7multiplikator_amd import _lib
    return _lib.load()


def host(t):
    torch.cuda.synchronize()
    return t.cpu().numpy()


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32 if a.dtype == np.float32 else np.uint8)


@pytest.mark.parametrize("gs", [32, 64])
def test_swiglu_q8_codes_beside_up_in_one_arena(L, oracle, gs):
    """gate | up | codes | scales carved from one allocation: the codes start at the byte after up."""
    rows, hidden = 64, 8192
    n = rows * hidden
    g = C.normal(41, (rows, hidden), 1.5)
    u = C.normal(42, (rows, hidden), 1.5)
    arena = torch.empty(2 * n * 4 + n + n // gs * 4, dtype=torch.uint8, device="cuda")
    gate = arena[: n * 4].view(torch.float32)
    up = arena[n * 4: 2 * n * 4].view(torch.float32)
    codes = arena[2 * n * 4: 2 * n * 4 + n]
    scales = arena[2 * n * 4 + n:].view(torch.float32)
    gate.copy_(torch.from_numpy(g.reshape(-1)))
    up.copy_(torch.from_numpy(u.reshape(-1)))
    rc = L.v7g_swiglu_q8(codes.data_ptr(), scales.data_ptr(), gate.data_ptr(), up.data_ptr(), rows, hidden, gs)
    assert rc == 0
    wq, ws = oracle.swiglu_q8(g, u, gs)
    assert np.array_equal(host(codes).view(np.int8), wq.reshape(-1))
    assert np.array_equal(bits(host(scales)), bits(ws.reshape(-1)))
    assert np.array_equal(host(up), u.reshape(-1)) and np.array_equal(host(gate), g.reshape(-1))


def test_swiglu_q8_over_up_is_refused_and_touches_nothing(L):
    rows, hidden = 8, 1024
    g = torch.randn(rows, hidden, device="cuda")
    u = torch.randn(rows, hidden, device="cuda")
    before = u.clone()
    L.v7g_clear_last_error()
    rc = L.v7g_swiglu_q8(u.data_ptr(), u.data_ptr() + rows * hidden, g.data_ptr(), u.data_ptr(), rows, hidden, 64)
    assert rc == 7 and L.v7g_get_last_error() == 7
    L.v7g_clear_last_error()
    assert torch.equal(u, before)


def test_fused_add_rmsnorm_out_over_add(L, oracle):
    """o == add: each row's add is read by its own workgroup before o is written."""
    r = C.normal(51, (128, 4096))
    a = C.normal(52, (128, 4096))
    w = C.norm_weight(53, 4096)
    want_o, want_r = oracle.fused_add_rmsnorm(r, a, w, 1e-6)
    rt, at, wt = (torch.from_numpy(x).cuda() for x in (r, a, w))
    assert L.v7g_fused_add_rmsnorm(at.data_ptr(), rt.data_ptr(), at.data_ptr(), wt.data_ptr(), 128, 4096, 1e-6) == 0
    assert np.array_equal(bits(host(at)), bits(want_o)) and np.array_equal(bits(host(rt)), bits(want_r))


def test_swiglu_out_over_up_and_add_inplace_doubling(L, oracle):
    g = C.normal(61, (256, 6144), 1.5)
    u = C.normal(62, (256, 6144), 1.5)
    gt, ut = torch.from_numpy(g).cuda(), torch.from_numpy(u).cuda()
    assert L.v7g_swiglu_f32(ut.data_ptr(), gt.data_ptr(), ut.data_ptr(), g.size) == 0
    assert np.array_equal(bits(host(ut)), bits(oracle.swiglu(g, u)))
    xt = torch.from_numpy(g).cuda()
    assert L.v7g_add_inplace(xt.data_ptr(), xt.data_ptr(), g.size) == 0
    assert np.array_equal(bits(host(xt)), bits(oracle.add_inplace(g, g)))


def test_qk_heads_inside_one_qkv_row_pass(L, oracle):
    """Q, K and V heads interleaved in one fused QKV row (same token stride) are apart: accepted, bit-exact."""
    T, HD, NQ, NK = 64, 128, 8, 2
    W = (NQ + 2 * NK) * HD
    qkv = C.normal(71, (T, W))
    qw, kw = C.norm_weight(72, HD), C.norm_weight(73, HD)
    ct, st = oracle.rope_tables(T, HD, 1e6)
    pos = np.arange(T, dtype=np.int32)
    d = torch.from_numpy(qkv).cuda()
    qwt, kwt, ctt, stt = (torch.from_numpy(x).cuda() for x in (qw, kw, ct, st))
    rc = L.v7g_qk_rmsnorm_rope(d.data_ptr(), W, NQ, qwt.data_ptr(), d.data_ptr() + NQ * HD * 4, W, NK, kwt.data_ptr(),
                               T, HD, ctt.data_ptr(), stt.data_ptr(), None, 0, HD // 2, T, 1e-6)
    assert rc == 0
    got = host(d)
    wq = oracle.rmsnorm_rope(qkv[:, : NQ * HD].reshape(T, NQ, HD), qw, ct, st, pos, 1e-6)
    wk = oracle.rmsnorm_rope(qkv[:, NQ * HD:(NQ + NK) * HD].reshape(T, NK, HD), kw, ct, st, pos, 1e-6)
    assert np.array_equal(bits(got[:, : NQ * HD]), bits(wq.reshape(T, -1)))
    assert np.array_equal(bits(got[:, NQ * HD:(NQ + NK) * HD]), bits(wk.reshape(T, -1)))
    assert np.array_equal(got[:, (NQ + NK) * HD:], qkv[:, (NQ + NK) * HD:])
