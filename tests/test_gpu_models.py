"""The four per-layer kernels at the model shapes of the load test's `models` mode (csrc/v7g_loadtest.cpp
kModels: the published widths, head counts, head_dims, QKV bias / Q-K norm and intermediate sizes of fourteen
open-weight models), bit for bit against the oracle: the Q8 embedding gather (a small vocabulary at the model's
width), add+RMSNorm over the width, the Q/K step inside the fused QKV row (RMSNorm+RoPE with Q/K norms, else RoPE
only with the QKV bias added to Q, K and V first where the model has one, and the K/V binary16 cache rows), and
SwiGLU -> Q8 over the intermediate size (32-element groups).  11 tokens, 2053 for the Q/K step.  Every
shape-specific launch the library picks for these shapes (the fixed-length add+RMSNorm rows, embedding blocks sized
to the row, the bias through the weight registers, 16 lanes per head at head_dim 256, the flat layout for head
counts that are not multiples of a wave's heads) runs here."""
from __future__ import annotations

import numpy as np
import pytest

from tests import common as C

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

# name, dim, q heads, kv heads, head_dim, hidden, Q/K norm, QKV bias (the load test's model table)
MODELS = [
    ("Qwen2.5-0.5B", 896, 14, 2, 64, 4864, False, True),
    ("Qwen3-0.6B", 1024, 16, 8, 128, 3072, True, False),
    ("Gemma-3-1B", 1152, 4, 1, 256, 6912, True, False),
    ("Llama-3.2-1B", 2048, 32, 8, 64, 8192, False, False),
    ("TinyLlama-1.1B", 2048, 32, 4, 64, 5632, False, False),
    ("Qwen2.5-1.5B", 1536, 12, 2, 128, 8960, False, True),
    ("Gemma-2-2B", 2304, 8, 4, 256, 9216, False, False),
    ("Qwen3-4B", 2560, 32, 8, 128, 9728, True, False),
    ("Phi-3-mini", 3072, 32, 32, 96, 8192, False, False),
    ("Qwen2.5-7B", 3584, 28, 4, 128, 18944, False, True),
    ("Gemma-3-12B", 3840, 16, 8, 256, 15360, True, False),
    ("Llama-3-8B", 4096, 32, 8, 128, 14336, False, False),
    ("Qwen3-14B", 5120, 40, 8, 128, 17408, True, False),
    ("Llama-3-70B", 8192, 64, 8, 128, 28672, False, False),
]
T_ROWS = 11
T_QKV = 2053  # the Q/K/V stage over more than 2048 tokens: head counts that are not multiples of 8 take the flat layout


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
    return t.detach().cpu().numpy()


def same(a, b):
    a, b = np.asarray(a), np.asarray(b)
    if a.dtype == np.float32:
        a, b = a.view(np.uint32), b.astype(np.float32).view(np.uint32)
    return a.shape == b.shape and np.array_equal(a, b)


@pytest.mark.parametrize("name,dim,nq,nkv,hd,hidden,qk_norm,bias", MODELS, ids=[m[0] for m in MODELS])
def test_model_layer_kernels(ops, oracle, name, dim, nq, nkv, hd, hidden, qk_norm, bias):
    seed = dim + hd
    T = T_ROWS
    # Q8 embedding gather at the model's width (a 300-row table; the kernel's blocks depend on the width only)
    tq, ts = C.q8_table(seed, 300, dim)
    ids = C.rng(seed).integers(0, 300, T).astype(np.int32)
    assert same(host(ops.embedding_gather_q8(dev(ids), dev(tq), dev(ts))), oracle.embedding_gather(ids, tq, ts, dim))

    # add+RMSNorm over the width
    r, a = C.normal(seed + 1, (T, dim)), C.normal(seed + 2, (T, dim))
    w = C.norm_weight(seed + 3, dim)
    want_o, want_r = oracle.fused_add_rmsnorm(r, a, w, 1e-6)
    rt = dev(r)
    got_o = ops.fused_add_rmsnorm(rt, dev(a), dev(w), eps=1e-6)
    assert same(host(rt), want_r) and same(host(got_o), want_o), "add+RMSNorm"

    # the Q/K step inside the fused QKV row, with the K/V cache rows
    T = T_QKV
    qkv = C.normal(seed + 4, (T, (nq + 2 * nkv) * hd))
    qw, kw = C.norm_weight(seed + 5, hd), C.norm_weight(seed + 6, hd)
    qb = C.normal(seed + 7, nq * hd, 0.5) if bias else None
    kb = C.normal(seed + 8, nkv * hd, 0.5) if bias else None
    vb = C.normal(seed + 9, nkv * hd, 0.5) if bias else None
    ct, st = oracle.rope_tables(T + 4, hd, 1e6)
    pos = (np.arange(T) + 3).astype(np.int32)
    pos[[2, 1000]] = 0
    q_np = qkv[:, :nq * hd].reshape(T, nq, hd)
    k_np = qkv[:, nq * hd:(nq + nkv) * hd].reshape(T, nkv, hd)
    v_np = qkv[:, (nq + nkv) * hd:].reshape(T, nkv, hd)
    wq, wk, wv, wkc, wvc = oracle.qkv_stage(q_np, k_np, v_np, qw if qk_norm else None, kw if qk_norm else None, qb,
                                            kb, vb, ct, st, pos, 1e-6)
    t = dev(qkv)
    q = t[:, :nq * hd].view(T, nq, hd)
    k = t[:, nq * hd:(nq + nkv) * hd].view(T, nkv, hd)
    v = t[:, (nq + nkv) * hd:].view(T, nkv, hd)
    kc = torch.zeros((T, nkv, hd), dtype=torch.float16, device="cuda")
    vc = torch.zeros((T, nkv, hd), dtype=torch.float16, device="cuda")
    d = lambda x: None if x is None else dev(x)  # noqa: E731
    ops.qkv_rope_stage(q, k, v, dev(ct), dev(st), positions=dev(pos), eps=1e-6,
                       q_norm_weight=d(qw) if qk_norm else None, k_norm_weight=d(kw) if qk_norm else None,
                       q_bias=d(qb), k_bias=d(kb), v_bias=d(vb), k_cache=kc, v_cache=vc)
    out = host(t)
    assert same(out[:, :nq * hd].reshape(T, nq, hd), wq), "q"
    assert same(out[:, nq * hd:(nq + nkv) * hd].reshape(T, nkv, hd), wk), "k"
    assert same(out[:, (nq + nkv) * hd:].reshape(T, nkv, hd), wv), "v"
    assert same(host(kc).view(np.uint16), wkc) and same(host(vc).view(np.uint16), wvc), "k/v cache"
    if qk_norm:  # the chain's own entry (no bias, no cache) on the same row
        t = dev(qkv)
        q = t[:, :nq * hd].view(T, nq, hd)
        k = t[:, nq * hd:(nq + nkv) * hd].view(T, nkv, hd)
        ops.qk_rmsnorm_rope(q, k, dev(qw), dev(kw), dev(ct), dev(st), positions=dev(pos), eps=1e-6)
        out = host(t)
        assert same(out[:, :nq * hd].reshape(T, nq, hd), oracle.rmsnorm_rope(q_np, qw, ct, st, pos, 1e-6)), "q"
        assert same(out[:, nq * hd:(nq + nkv) * hd].reshape(T, nkv, hd),
                    oracle.rmsnorm_rope(k_np, kw, ct, st, pos, 1e-6)), "k"

    # SwiGLU -> Q8 over the intermediate size
    T = T_ROWS
    g, u = C.normal(seed + 10, (T, hidden), 1.5), C.normal(seed + 11, (T, hidden), 1.5)
    want_q, want_s = oracle.swiglu_q8(g, u, 32)
    got_q, got_s = ops.swiglu_q8(dev(g), dev(u), gs=32)
    assert same(host(got_q), want_q) and same(host(got_s), want_s), "SwiGLU -> Q8"
