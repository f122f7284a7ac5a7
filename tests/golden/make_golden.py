"""Writes tests/golden/fixtures.npz: small seeded inputs and the oracle's outputs for every kernel of the path.

    python tests/golden/make_golden.py

The reference holds no golden vectors for these kernels (its validators draw inputs from libc rand()
at run time, tools/kt_utils.h:117-127), so these fixtures come from the oracle (oracle/), whose
restatement is pinned by tests/test_oracle.py.  tests/test_golden.py checks that the oracle still
reproduces them (CPU) and that the GPU kernels produce them (GPU).  Inputs use numpy's Philox
generator, so the file is the same on every platform.
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import oracle as O  # noqa: E402
from tests import common as C  # noqa: E402


def main():
    f = {}
    # a1 fused add + RMSNorm: dims with and without leftover blocks, eps 1e-6
    for dim in (40, 256):
        r = C.normal(1000 + dim, (3, dim))
        a = C.normal(2000 + dim, (3, dim))
        w = C.norm_weight(3000 + dim, dim)
        o, rr = O.fused_add_rmsnorm(r, a, w, 1e-6)
        f.update({f"arn{dim}_residual": r, f"arn{dim}_add": a, f"arn{dim}_weight": w, f"arn{dim}_o": o,
                  f"arn{dim}_residual_out": rr})
    # a3 RMSNorm + RoPE: 4 tokens (pos 0, 1, 9, 31) x 3 heads, hd 128 (register rotation) and 96 (LDS rotation)
    for hd in (128, 96):
        x = C.normal(4000 + hd, (4, 3, hd))
        w = C.norm_weight(5000 + hd, hd)
        ct, st = O.rope_tables(32, hd, 1e6)
        pos = np.array([0, 1, 9, 31], np.int32)
        f.update({f"rope{hd}_x": x, f"rope{hd}_w": w, f"rope{hd}_cos": ct, f"rope{hd}_sin": st, f"rope{hd}_pos": pos,
                  f"rope{hd}_out": O.rmsnorm_rope(x, w, ct, st, pos, 1e-6)})
    # a6 SwiGLU f32 (odd length: vector body + tail)
    g = C.normal(6001, 1027, 1.5)
    u = C.normal(6002, 1027, 1.5)
    f.update({"swiglu_gate": g, "swiglu_up": u, "swiglu_out": O.swiglu(g, u)})
    # a7 quantize: GS 64 with a 36-element tail group per row, GS 32 on a ragged-free row, and a zero group
    x = C.normal(7001, (2, 100), 3.0)
    q, s = O.quantize(x, 64)
    f.update({"q64_x": x, "q64_codes": q, "q64_scales": s})
    x = C.normal(7002, (2, 256), 3.0)
    x[1, 32:64] = 0.0
    q, s = O.quantize(x, 32)
    f.update({"q32_x": x, "q32_codes": q, "q32_scales": s})
    # a8 SwiGLU -> Q8, GS 32 and 64
    g = C.normal(8001, (2, 512), 1.5)
    u = C.normal(8002, (2, 512), 1.5)
    for gs in (32, 64):
        q, s = O.swiglu_q8(g, u, gs)
        f.update({f"sq8_{gs}_codes": q, f"sq8_{gs}_scales": s})
    f.update({"sq8_gate": g, "sq8_up": u})
    # a9 Q8 embedding gather
    tq, ts = C.q8_table(9001, 40, 128)
    ids = np.array([0, 39, 17, 17, 5], np.int32)
    f.update({"emb_table_q": tq, "emb_table_s": ts, "emb_ids": ids, "emb_out": O.embedding_gather(ids, tq, ts, 128)})
    path = os.path.join(HERE, "fixtures.npz")
    np.savez_compressed(path, **f)
    print(path, os.path.getsize(path), "bytes,", len(f), "arrays")


if __name__ == "__main__":
    main()
