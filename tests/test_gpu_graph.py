"""The batched entries under HIP graph capture: the per-layer chain (Q8 embedding gather, add+RMSNorm,
Q/K RMSNorm+RoPE inside a fused QKV row, SwiGLU -> Q8) and the RMSNorm -> Q8 / K/V pack rows, captured once
with torch.cuda.graph on torch's capture stream (the library binds to the caller's current stream) and
replayed several times, with eager work between the replays (the in-place inputs restored, the outputs
cleared), each replay checked bit for bit against one eager pass of the same calls.  None of these entries
records a memset or allocates inside the capture.
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

    def step():
        ops.embedding_gather_q8(ids, tq, ts, out=emb)
        ops.fused_add_rmsnorm(residual, add, w, eps=1e-6, out=normed)
        ops.qk_rmsnorm_rope(q, k, qw, kw, ct, st, positions=pos, eps=1e-6)
        ops.swiglu_q8(gate, up, gs=GS, out_q=codes, out_s=scales)
        ops.rmsnorm_quantize(x_nq, w, eps=1e-6, gs=64, out_q=nq_codes, out_s=nq_scales)
        ops.kv_pack_f16_kv(qkv[:, NQ * HD:(NQ + NKV) * HD], v, k_out=kc, v_out=vc)

    outs = (emb, residual, normed, qkv, codes, scales, nq_codes, nq_scales, kc, vc)

    def reset():
        residual.copy_(residual0)
        qkv.copy_(qkv0)
        for o in (emb, normed, scales, nq_scales):
            o.fill_(-1.0)
        for o in (codes, nq_codes):
            o.fill_(0)
        for o in (kc, vc):
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
            for o, w_, name in zip(outs, want, ("emb", "residual", "normed", "qkv", "codes", "scales", "nq codes",
                                                "nq scales", "k cache", "v cache")):
                assert np.array_equal(bits(o), w_), (replay, name)
    finally:
        # the library binds each host thread to the stream of its last call: back to the current stream
        from v7multiplikator_amd import _lib
        _lib.load().v7g_set_stream(torch.cuda.current_stream().cuda_stream)
