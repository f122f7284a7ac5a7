"""The batched entries and the drop-ins under HIP graph capture: the per-layer chain (Q8 embedding gather, add+RMSNorm,
Q/K RMSNorm+RoPE inside a fused QKV row, SwiGLU -> Q8) and the widened rows (RMSNorm -> Q8, the K/V pack, the Q/K/V
stage with the QKV bias and both cache rows in the flat layout, add -> RMSNorm -> Q8, add_inplace), captured once
with torch.cuda.graph on torch's capture stream (the library binds to the caller's current stream) and
replayed several times, with eager work between the replays (the in-place inputs restored, the outputs
cleared), each replay checked bit for bit against one eager pass of the same calls; and a one-token decode
step of reference-signature drop-in calls, captured the same way.  None of these entries records a memset or
allocates inside the capture.
"""
from __future__ import annotations

import numpy as np
import pytest

from tests import common as C

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

T, DIM, VOCAB, NQ, NKV, HD, HID, GS = 96, 512, 1000, 4, 2, 128, 1024, 32


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


def bits(t):
    a = t.detach().cpu().numpy()
    return a.view(np.uint32) if a.dtype == np.float32 else a


def test_chain_replays_from_a_hip_graph(ops, oracle):
    tq, ts = C.q8_table(11, VOCAB, DIM)
    ids = dev(C.rng(12).integers(0, VOCAB, T).astype(np.int32))
    tq, ts = dev(tq), dev(ts)
    residual0 = dev(C.normal(13, (T, DIM)))
    add = dev(C.normal(14, (T, DIM)))
    w = dev(C.norm_weight(15, DIM))
    qkv0 = dev(C.normal(16, (T, (NQ + 2 * NKV) * HD)))
    qw, kw = dev(C.norm_weight(17, HD)), dev(C.norm_weight(18, HD))
    ct, st = oracle.rope_tables(T, HD, 1e6)
    ct, st = dev(ct), dev(st)
    pos = torch.arange(T, dtype=torch.int32, device="cuda")
    gate = dev(C.normal(19, (T, HID), 1.5))
    up = dev(C.normal(20, (T, HID), 1.5))
    x_nq = dev(C.normal(21, (T, DIM), 2.0))

    # static buffers the graph reads and writes
    emb = torch.empty((T, DIM), device="cuda")
    residual = residual0.clone()
    normed = torch.empty((T, DIM), device="cuda")
    qkv = qkv0.clone()
    codes = torch.empty((T, HID), dtype=torch.int8, device="cuda")
    scales = torch.empty((T, HID // GS), device="cuda")
    nq_codes = torch.empty((T, DIM), dtype=torch.int8, device="cuda")
    nq_scales = torch.empty((T, DIM // 64), device="cuda")
    kc = torch.empty((T, NKV * HD), dtype=torch.float16, device="cuda")
    vc = torch.empty((T, NKV * HD), dtype=torch.float16, device="cuda")
    q = qkv[:, :NQ * HD].view(T, NQ, HD)
    k = qkv[:, NQ * HD:(NQ + NKV) * HD].view(T, NKV, HD)
    v = qkv[:, (NQ + NKV) * HD:]
    # the Q/K/V stage with the QKV bias and both cache rows over 1030 tokens of 6 + 1 + 1 heads: the flat layout
    T2, NQ2, NKV2 = 1030, 6, 1
    qkv2_0 = dev(C.normal(22, (T2, (NQ2 + 2 * NKV2) * HD)))
    bias2 = dev(C.normal(23, (NQ2 + 2 * NKV2) * HD, 0.5))
    ct2, st2 = oracle.rope_tables(T2 + 2, HD, 1e6)
    ct2, st2 = dev(ct2), dev(st2)
    pos2 = torch.arange(T2, dtype=torch.int32, device="cuda")
    qkv2 = qkv2_0.clone()
    kc2 = torch.empty((T2, NKV2, HD), dtype=torch.float16, device="cuda")
    vc2 = torch.empty((T2, NKV2, HD), dtype=torch.float16, device="cuda")
    q2 = qkv2[:, :NQ2 * HD].view(T2, NQ2, HD)
    k2 = qkv2[:, NQ2 * HD:(NQ2 + NKV2) * HD].view(T2, NKV2, HD)
    v2 = qkv2[:, (NQ2 + NKV2) * HD:].view(T2, NKV2, HD)
    # add -> RMSNorm -> Q8 (residual updated in place) and add_inplace
    res3_0 = dev(C.normal(24, (T, DIM)))
    res3 = res3_0.clone()
    aq_codes = torch.empty((T, DIM), dtype=torch.int8, device="cuda")
    aq_scales = torch.empty((T, DIM // 64), device="cuda")
    xa0 = dev(C.normal(25, (T, DIM)))
    xa = xa0.clone()

    def step():
        ops.embedding_gather_q8(ids, tq, ts, out=emb)
        ops.fused_add_rmsnorm(residual, add, w, eps=1e-6, out=normed)
        ops.qk_rmsnorm_rope(q, k, qw, kw, ct, st, positions=pos, eps=1e-6)
        ops.swiglu_q8(gate, up, gs=GS, out_q=codes, out_s=scales)
        ops.rmsnorm_quantize(x_nq, w, eps=1e-6, gs=64, out_q=nq_codes, out_s=nq_scales)
        ops.kv_pack_f16_kv(qkv[:, NQ * HD:(NQ + NKV) * HD], v, k_out=kc, v_out=vc)
        ops.qkv_rope_stage(q2, k2, v2, ct2, st2, positions=pos2, eps=1e-6, q_bias=bias2[:NQ2 * HD],
                           k_bias=bias2[NQ2 * HD:(NQ2 + NKV2) * HD], v_bias=bias2[(NQ2 + NKV2) * HD:], k_cache=kc2,
                           v_cache=vc2)
        ops.add_rmsnorm_quantize(res3, add, w, eps=1e-6, gs=64, out_q=aq_codes, out_s=aq_scales)
        ops.add_inplace(xa, add)

    outs = (emb, residual, normed, qkv, codes, scales, nq_codes, nq_scales, kc, vc, qkv2, kc2, vc2, res3, aq_codes,
            aq_scales, xa)
    names = ("emb", "residual", "normed", "qkv", "codes", "scales", "nq codes", "nq scales", "k cache", "v cache",
             "qkv stage", "qkv stage k cache", "qkv stage v cache", "add+norm->q8 residual", "add+norm->q8 codes",
             "add+norm->q8 scales", "add_inplace")

    def reset():
        residual.copy_(residual0)
        qkv.copy_(qkv0)
        qkv2.copy_(qkv2_0)
        res3.copy_(res3_0)
        xa.copy_(xa0)
        for o in (emb, normed, scales, nq_scales, aq_scales):
            o.fill_(-1.0)
        for o in (codes, nq_codes, aq_codes):
            o.fill_(0)
        for o in (kc, vc, kc2, vc2):
            o.fill_(0)

    # one eager pass: the expected outputs
    reset()
    step()
    torch.cuda.synchronize()
    want = [bits(o) for o in outs]

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        reset()
        step()  # warm-up on the side stream before capture
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()

    g = torch.cuda.CUDAGraph()
    reset()
    torch.cuda.synchronize()
    try:
        with torch.cuda.graph(g):
            step()
        torch.cuda.synchronize()

        for replay in range(4):
            reset()  # eager work between the replays
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            for o, w_, name in zip(outs, want, names):
                assert np.array_equal(bits(o), w_), (replay, name)
    finally:
        # the library binds each host thread to the stream of its last call: back to the current stream
        from v7multiplikator_amd import _lib
        _lib.load().v7g_set_stream(torch.cuda.current_stream().cuda_stream)


def test_dropin_decode_step_replays_from_a_hip_graph(ops, oracle):
    """A one-token decode step made of the reference-signature drop-ins (ms_abi, through tests/libdropin_shim.so,
    as a v7 host calls them): the embedding row, add+RMSNorm, Q and K RMSNorm+RoPE at position 37, the K row
    packed to binary16, SwiGLU -> Q8 of the FFN row.  Captured once on torch's capture stream (bound with
    v7g_set_stream inside the capture), replayed four times with eager work between, each replay equal to one
    eager pass bit for bit: one graph launch instead of six kernel launches."""
    import ctypes
    import os

    from v7multiplikator_amd import _lib
    shim_path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libdropin_shim.so")
    if not os.path.exists(shim_path):
        pytest.fail(f"{shim_path} is missing: run __graft_entry__.build()")
    S = ctypes.CDLL(shim_path)
    vp, i = ctypes.c_void_p, ctypes.c_int
    S.shim_embedding_row.argtypes = [vp, i, i, vp, vp]
    S.shim_fused_add_rmsnorm.argtypes = [vp, vp, vp, vp, i]
    S.shim_rmsnorm_rope_heads.argtypes = [vp, i, i, vp, vp, vp, i, i]
    S.shim_kv_pack_f16.argtypes = [vp, vp, i]
    S.shim_swiglu_quantize_row.argtypes = [vp, vp, vp, vp, i]
    L = _lib.load()
    L.v7g_set_rms_eps(ctypes.c_float(1e-6))
    POS = 37
    tq, ts = C.q8_table(31, VOCAB, DIM)
    tq, ts = dev(tq), dev(ts)
    residual0 = dev(C.normal(32, DIM))
    w = dev(C.norm_weight(33, DIM))
    qkv0 = dev(C.normal(34, (NQ + 2 * NKV) * HD))
    qw, kw = dev(C.norm_weight(35, HD)), dev(C.norm_weight(36, HD))
    ct, st = oracle.rope_tables(64, HD, 1e6)
    ct, st = dev(ct), dev(st)
    gate, up = dev(C.normal(37, HID, 1.5)), dev(C.normal(38, HID, 1.5))

    emb = torch.empty(DIM, device="cuda")
    residual = residual0.clone()
    normed = torch.empty(DIM, device="cuda")
    qkv = qkv0.clone()
    kc = torch.empty(NKV * HD, dtype=torch.float16, device="cuda")
    codes = torch.empty(HID, dtype=torch.int8, device="cuda")
    scales = torch.empty(HID // 64, device="cuda")
    p = lambda t: t.data_ptr()  # noqa: E731

    def step():
        L.v7g_set_stream(torch.cuda.current_stream().cuda_stream)
        S.shim_embedding_row(p(emb), 123, DIM, p(tq), p(ts))
        S.shim_fused_add_rmsnorm(p(normed), p(residual), p(emb), p(w), DIM)
        S.shim_rmsnorm_rope_heads(p(qkv), NQ, HD, p(qw), p(ct), p(st), POS, HD // 2)
        S.shim_rmsnorm_rope_heads(p(qkv) + NQ * HD * 4, NKV, HD, p(kw), p(ct), p(st), POS, HD // 2)
        S.shim_kv_pack_f16(p(kc), p(qkv) + NQ * HD * 4, NKV * HD)
        S.shim_swiglu_quantize_row(p(codes), p(gate), p(up), p(scales), HID)

    outs = (emb, residual, normed, qkv, kc, codes, scales)

    def reset():
        residual.copy_(residual0)
        qkv.copy_(qkv0)
        for o in (emb, normed, scales):
            o.fill_(-1.0)
        codes.fill_(0)
        kc.fill_(0)

    L.v7g_clear_last_error()
    reset()
    step()
    torch.cuda.synchronize()
    assert L.v7g_get_last_error() == 0
    want = [bits(o) for o in outs]
    # the eager pass against the oracle: the decode step's results are the reference's
    r_new = C.normal(32, DIM) + oracle.embedding_gather(np.array([123], np.int32), host_np(tq), host_np(ts), DIM)[0]
    assert np.array_equal(want[1], r_new.astype(np.float32).view(np.uint32))

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        reset()
        step()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()

    g = torch.cuda.CUDAGraph()
    reset()
    torch.cuda.synchronize()
    try:
        with torch.cuda.graph(g):
            step()
        torch.cuda.synchronize()
        for replay in range(4):
            reset()
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            for o, w_, name in zip(outs, want, ("emb", "residual", "normed", "qkv", "k cache", "codes", "scales")):
                assert np.array_equal(bits(o), w_), (replay, name)
        assert L.v7g_get_last_error() == 0
    finally:
        L.v7g_set_stream(torch.cuda.current_stream().cuda_stream)
        L.v7g_clear_last_error()


def host_np(t):
    return t.detach().cpu().numpy()
