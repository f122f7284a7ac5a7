"""Committed golden vectors (tests/golden/fixtures.npz, written by tests/golden/make_golden.py).

CPU: the oracle still reproduces every fixture bit for bit (a change to the restatement shows here).
GPU: the kernels produce every fixture bit for bit, without running the oracle.
"""
from __future__ import annotations

import os

import numpy as np
import pytest

FIX = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "fixtures.npz")


@pytest.fixture(scope="module")
def fx():
    with np.load(FIX, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def same(a, b):
    a, b = np.asarray(a), np.asarray(b)
    if a.shape != b.shape:
        return False
    if a.dtype.kind == "f":
        return np.array_equal(a.view(np.uint32), b.view(np.uint32))
    return np.array_equal(a, b)


# --------------------------------------------------------------------------- CPU: oracle vs fixtures

def test_oracle_reproduces_fixtures(fx, oracle):
    for dim in (40, 256):
        o, r = oracle.fused_add_rmsnorm(fx[f"arn{dim}_residual"], fx[f"arn{dim}_add"], fx[f"arn{dim}_weight"], 1e-6)
        assert same(o, fx[f"arn{dim}_o"]) and same(r, fx[f"arn{dim}_residual_out"])
    for hd in (128, 96):
        out = oracle.rmsnorm_rope(fx[f"rope{hd}_x"], fx[f"rope{hd}_w"], fx[f"rope{hd}_cos"], fx[f"rope{hd}_sin"],
                                  fx[f"rope{hd}_pos"], 1e-6)
        assert same(out, fx[f"rope{hd}_out"])
        c, s = oracle.rope_tables(32, hd, 1e6)
        assert same(c, fx[f"rope{hd}_cos"]) and same(s, fx[f"rope{hd}_sin"])
    assert same(oracle.swiglu(fx["swiglu_gate"], fx["swiglu_up"]), fx["swiglu_out"])
    q, s = oracle.quantize(fx["q64_x"], 64)
    assert same(q, fx["q64_codes"]) and same(s, fx["q64_scales"])
    q, s = oracle.quantize(fx["q32_x"], 32)
    assert same(q, fx["q32_codes"]) and same(s, fx["q32_scales"])
    for gs in (32, 64):
        q, s = oracle.swiglu_q8(fx["sq8_gate"], fx["sq8_up"], gs)
        assert same(q, fx[f"sq8_{gs}_codes"]) and same(s, fx[f"sq8_{gs}_scales"])
    assert same(oracle.embedding_gather(fx["emb_ids"], fx["emb_table_q"], fx["emb_table_s"], 128), fx["emb_out"])


def test_fixture_closed_forms(fx):
    """Facts of the fixtures that hold independently of the oracle."""
    # embedding: exact int8 -> f32 times the 64-code group scale
    tq, ts, ids = fx["emb_table_q"], fx["emb_table_s"], fx["emb_ids"]
    want = tq[ids].astype(np.float32) * np.repeat(ts.reshape(40, 2)[ids], 64, axis=1)
    assert same(fx["emb_out"], want.astype(np.float32))
    # quantizer: the zero group's scale is exactly 2^-126 and its codes are 0; absmax codes are +-127
    assert fx["q32_scales"][1, 1] == np.float32(2.0 ** -126) and not fx["q32_codes"][1, 32:64].any()
    assert np.abs(fx["q64_codes"].astype(int)).max() == 127
    # residual update is one binary32 add per element
    assert same(fx["arn40_residual_out"], (fx["arn40_residual"] + fx["arn40_add"]).astype(np.float32))
    # RoPE at pos 0 leaves the rotation out: both halves keep the normalised values (no mixing)
    x0 = fx["rope128_x"][0].astype(np.float64)
    n0 = x0 / np.sqrt(np.mean(x0 * x0, axis=-1, keepdims=True) + 1e-6) * fx["rope128_w"]
    assert np.max(np.abs(fx["rope128_out"][0] - n0)) < 1e-5


# --------------------------------------------------------------------------- GPU: kernels vs fixtures

@pytest.mark.gpu
def test_gpu_reproduces_fixtures(fx):
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a visible MI355X")
    from v7multiplikator_amd import ops

    d = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    h = lambda t: (torch.cuda.synchronize(), t.cpu().numpy())[1]  # noqa: E731
    for dim in (40, 256):
        r = d(fx[f"arn{dim}_residual"])
        o = ops.fused_add_rmsnorm(r, d(fx[f"arn{dim}_add"]), d(fx[f"arn{dim}_weight"]), eps=1e-6)
        assert same(h(o), fx[f"arn{dim}_o"]) and same(h(r), fx[f"arn{dim}_residual_out"]), dim
    for hd in (128, 96):
        b = d(fx[f"rope{hd}_x"])
        ops.rmsnorm_rope_heads(b, d(fx[f"rope{hd}_w"]), d(fx[f"rope{hd}_cos"]), d(fx[f"rope{hd}_sin"]),
                               positions=d(fx[f"rope{hd}_pos"]), eps=1e-6)
        assert same(h(b), fx[f"rope{hd}_out"]), hd
    assert same(h(ops.swiglu(d(fx["swiglu_gate"]), d(fx["swiglu_up"]))), fx["swiglu_out"])
    q, s = ops.quantize_q8(d(fx["q64_x"]), gs=64)
    assert same(h(q), fx["q64_codes"]) and same(h(s), fx["q64_scales"])
    q, s = ops.quantize_q8(d(fx["q32_x"]), gs=32)
    assert same(h(q), fx["q32_codes"]) and same(h(s), fx["q32_scales"])
    for gs in (32, 64):
        q, s = ops.swiglu_q8(d(fx["sq8_gate"]), d(fx["sq8_up"]), gs=gs)
        assert same(h(q), fx[f"sq8_{gs}_codes"]) and same(h(s), fx[f"sq8_{gs}_scales"]), gs
    out = ops.embedding_gather_q8(d(fx["emb_ids"]), d(fx["emb_table_q"]), d(fx["emb_table_s"]))
    assert same(h(out), fx["emb_out"])
