#!/usr/bin/env python3
"""Benchmark of the fused per-layer kernels on one MI355X.

Workload (one "step"): the per-layer elementwise chain at the Qwen3-8B shape
with T = 8192 tokens, every input resident in HBM:
  a. Q8 embedding gather of 8192 ids from a 151936 x 4096 int8 table (f32 scales, 64-code groups)
  b. fused residual-add + RMSNorm over [8192, 4096], eps 1e-6
  c. RMSNorm + RoPE over 32 Q and 8 KV heads (head_dim 128, theta 1e6, positions 0..T-1),
     Q/K inside a fused QKV row [8192, 6144] as the engine lays them out
  d. SwiGLU -> Q8 over gate/up [8192, 12288], 32-element blocks
Synthetic data: inputs drawn on the device from a seeded generator
(x, residual ~N(0,1); weights 1+N(0,0.1); gate/up ~N(0,1.5); codes uniform in
[-127,127], scales U(0.001,0.02)).

Reported value: whole-chain algorithmic bytes (every tensor read once and
written once) / wall time, in GB/s.  Per-kernel durations come from HIP events
bound to the kernels' own dispatch timestamps on the launch stream inside the
timed region; `roofline` reports the dominant kernel (SwiGLU -> Q8) against the
8 TB/s HBM peak.  `cpu_baseline`
times the AVX2 restatement of the reference kernels on the host cores, driven
per token row as the reference engine drives them, on a bounded sample of the
same workload; that leg also checks the GPU outputs of the sample bit for bit.
With V7_REF_SO naming a libv7_threading.so built by the reference's own
Makefile (nasm), `cpu_baseline.reference` adds that library's two exported
chain kernels (add+RMSNorm, Q/K RMSNorm+RoPE) on the same sample, beside the
restatement's same two kernels and checked against them bit for bit
(V7_REF_EPS: the eps its g_rms_eps global holds, 0 without its database init).

`rows` times the widened rows of the path at the same shapes, after the timed region and outside `value`
(RMSNorm -> Q8, its fused residual-add form, the K/V pack, the Q/K/V stage with binary16 cache rows, the
QKV-bias RoPE-only stage, add_inplace), each row's calls captured in a HIP graph and timed over one replay;
`cpu_baseline.rows` times the restatement of each row on the host, one call per token row over the host
threads, and checks the GPU's outputs for the same inputs bit for bit.

    python bench.py [--steps K] [--warmup W] [--cpu-seconds S] [--no-cpu] [--no-rows]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0

T = 8192
DIM = 4096
VOCAB = 151936
NQ, NKV, HD = 32, 8, 128
HIDDEN = 12288
GS = 32
THETA = 1e6
EPS = 1e-6

BYTES = {
    "embedding_gather_q8": T * 4 + T * DIM + T * (DIM // 64) * 4 + T * DIM * 4,
    "fused_add_rmsnorm": 4 * T * DIM * 4 + DIM * 4,
    "qk_rmsnorm_rope": 2 * T * (NQ + NKV) * HD * 4 + 2 * T * (HD // 2) * 4 + 2 * HD * 4,
    "swiglu_q8": 2 * T * HIDDEN * 4 + T * HIDDEN + T * (HIDDEN // GS) * 4,
}
DOMINANT = "swiglu_q8"

# The widened rows of the path at the same shapes (not part of `value`): bytes per call over T tokens.
QKV = (NQ + 2 * NKV) * HD
KVD = NKV * HD
ROW_BYTES = {
    "rmsnorm_quantize": T * DIM * 4 + T * DIM + T * (DIM // 64) * 4 + DIM * 4,
    "add_rmsnorm_quantize": 3 * T * DIM * 4 + T * DIM + T * (DIM // 64) * 4 + DIM * 4,
    "kv_pack_f16_kv": 2 * T * KVD * 4 + 2 * T * KVD * 2,
    "qkv_rope_stage": T * QKV * 4 + T * NQ * HD * 4 + 2 * T * KVD * 2 + 2 * T * (HD // 2) * 4 + 2 * HD * 4,
    "qkv_bias_rope_only": 2 * T * QKV * 4 + QKV * 4 + 2 * T * (HD // 2) * 4,
    "add_inplace": 3 * T * DIM * 4,
}
ROW_SHAPES = {
    "rmsnorm_quantize": "RMSNorm -> Q8 [8192, 4096], GS 64",
    "add_rmsnorm_quantize": "residual add then RMSNorm -> Q8 [8192, 4096], GS 64, one pass",
    "kv_pack_f16_kv": "K and V rows of the QKV row to binary16 cache rows, 8192 tokens x 1024, one launch",
    "qkv_rope_stage": "Q/K RMSNorm+RoPE 32 + 8 heads of 128, K/V to binary16 cache rows, f32 Q kept, 8192 tokens",
    "qkv_bias_rope_only": "QKV bias on Q, K, V then RoPE only on Q and K, 32 + 8 + 8 heads of 128, 8192 tokens",
    "add_inplace": "x += y over [8192, 4096]",
}
ROW_FORMS = {  # the restatement each row's CPU timing runs (oracle/)
    "rmsnorm_quantize": "AVX2 RMSNorm and Q8 quantizer restatement",
    "add_rmsnorm_quantize": "AVX2 vaddps, RMSNorm and Q8 quantizer restatement",
    "kv_pack_f16_kv": "F16C vcvtps2ph, the reference's instruction",
    "qkv_rope_stage": "AVX2 RMSNorm+RoPE restatement and the F16C pack",
    "qkv_bias_rope_only": "AVX2 vaddps bias and RoPE-only restatement (vmulps, vfnmadd231ps, vfmadd231ps)",
    "add_inplace": "AVX2 vaddps",
}
ROW_KINDS = {"rmsnorm_quantize": 0, "add_rmsnorm_quantize": 1, "kv_pack_f16_kv": 2, "qkv_rope_stage": 3,
             "qkv_bias_rope_only": 4, "add_inplace": 5}  # orc_rows_args.kind (oracle/v7_oracle.h)


def parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=200)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--seed", type=int, default=5)
    p.add_argument("--cpu-seconds", type=float, default=10.0)
    p.add_argument("--cpu-tokens", type=int, default=2048)
    p.add_argument("--no-cpu", action="store_true")
    p.add_argument("--no-rows", action="store_true", help="skip the widened rows (GPU pass and CPU leg)")
    p.add_argument("--copy-probe", action="store_true",
                   help="also run one 1 GiB torch copy (the scale reference for rocprofv3 --pmc byte counters)")
    return p.parse_args()


class Chain:
    """Device buffers of the chain and one launch per kernel.

    The activations are carved, in chain order, from one device arena, as an inference engine lays out
    its activation buffers; the weights and tables are separate allocations.  (With every activation a
    separate allocation, SwiGLU -> Q8 measured about 3% slower: how gate and up fall on the HBM
    channels against each other depends on where the allocator places them.)"""

    def __init__(self, torch, ops, seed, n_tokens=T):
        g = torch.Generator(device="cuda")
        g.manual_seed(seed)
        dev = "cuda"
        f32, i8 = torch.float32, torch.int8
        self.n = n_tokens
        layout = [("emb", (n_tokens, DIM), f32), ("residual", (n_tokens, DIM), f32), ("add", (n_tokens, DIM), f32),
                  ("normed", (n_tokens, DIM), f32), ("qkv", (n_tokens, (NQ + 2 * NKV) * HD), f32),
                  ("gate", (n_tokens, HIDDEN), f32), ("up", (n_tokens, HIDDEN), f32),
                  ("codes", (n_tokens, HIDDEN), i8), ("scales", (n_tokens, HIDDEN // GS), f32)]
        size = lambda shape, dt: -(-shape[0] * shape[1] * torch.empty(0, dtype=dt).element_size() // 256) * 256
        self.arena = torch.empty(sum(size(sh, dt) for _, sh, dt in layout), dtype=torch.uint8, device=dev)
        off = 0
        for name, shape, dt in layout:
            n = size(shape, dt)
            setattr(self, name, self.arena[off:off + n].view(dt)[:shape[0] * shape[1]].view(shape))
            off += n
        self.table_q = torch.randint(-127, 128, (VOCAB, DIM), generator=g, dtype=i8, device=dev)
        self.table_s = torch.empty(VOCAB * DIM // 64, dtype=f32, device=dev).uniform_(0.001, 0.02, generator=g)
        self.ids = torch.randint(0, VOCAB, (n_tokens,), generator=g, dtype=torch.int32, device=dev)
        self.residual.normal_(generator=g)
        self.add.normal_(generator=g)
        self.w_norm = 1.0 + 0.1 * torch.randn(DIM, generator=g, dtype=f32, device=dev)
        self.qkv.normal_(generator=g)
        self.q_w = 1.0 + 0.1 * torch.randn(HD, generator=g, dtype=f32, device=dev)
        self.k_w = 1.0 + 0.1 * torch.randn(HD, generator=g, dtype=f32, device=dev)
        self.cos, self.sin = ops.rope_tables(max(n_tokens, 1), HD, THETA)
        self.positions = torch.arange(n_tokens, dtype=torch.int32, device=dev)
        self.gate.normal_(generator=g).mul_(1.5)
        self.up.normal_(generator=g).mul_(1.5)
        self.ops = ops

    def q(self):
        return self.qkv[:, :NQ * HD].view(self.n, NQ, HD)

    def k(self):
        return self.qkv[:, NQ * HD:(NQ + NKV) * HD].view(self.n, NKV, HD)

    def launches(self):
        ops = self.ops
        return [
            ("embedding_gather_q8", lambda: ops.embedding_gather_q8(self.ids, self.table_q, self.table_s, out=self.emb)),
            ("fused_add_rmsnorm", lambda: ops.fused_add_rmsnorm(self.residual, self.add, self.w_norm, eps=EPS,
                                                                 out=self.normed)),
            ("qk_rmsnorm_rope", lambda: ops.qk_rmsnorm_rope(self.q(), self.k(), self.q_w, self.k_w, self.cos,
                                                            self.sin, positions=self.positions, eps=EPS)),
            ("swiglu_q8", lambda: ops.swiglu_q8(self.gate, self.up, gs=GS, out_q=self.codes, out_s=self.scales)),
        ]


class RowData:
    """Inputs of the widened rows over n tokens at the chain's shapes (the QKV rows carry Q, K and V heads)."""

    def __init__(self, torch, n, seed, device):
        g = torch.Generator(device=device)
        g.manual_seed(seed)
        f32 = torch.float32
        self.x = torch.randn((n, DIM), generator=g, dtype=f32, device=device)
        self.add = torch.randn((n, DIM), generator=g, dtype=f32, device=device)
        self.w = 1.0 + 0.1 * torch.randn(DIM, generator=g, dtype=f32, device=device)
        self.qkv = torch.randn((n, QKV), generator=g, dtype=f32, device=device)
        self.bias = 0.5 * torch.randn(QKV, generator=g, dtype=f32, device=device)
        self.q_w = 1.0 + 0.1 * torch.randn(HD, generator=g, dtype=f32, device=device)
        self.k_w = 1.0 + 0.1 * torch.randn(HD, generator=g, dtype=f32, device=device)
        self.positions = torch.arange(n, dtype=torch.int32, device=device)


ROW_SETS = 4  # buffer sets of the widened rows, used in turn


class Rows:
    """Device buffers of the widened rows and one launch per row.  ROW_SETS sets are used in turn, so that no
    call finds its inputs in the 256 MiB Infinity Cache: the smallest row, the K/V pack, touches about 100 MB
    per call (67 MB of K and V read, 33.5 MB of binary16 rows written), so four sets cycle through about
    400 MB before a set comes back (two sets, 200 MB, would fit in the cache)."""

    def __init__(self, torch, ops, chain, seed):
        self.ops, self.cos, self.sin = ops, chain.cos, chain.sin
        self.sets = []
        for i in range(ROW_SETS):
            d = RowData(torch, T, seed + 100 + i, "cuda")
            d.codes = torch.empty((T, DIM), dtype=torch.int8, device="cuda")
            d.scales = torch.empty((T, DIM // 64), dtype=torch.float32, device="cuda")
            d.kc = torch.empty((T, KVD), dtype=torch.float16, device="cuda")
            d.vc = torch.empty((T, KVD), dtype=torch.float16, device="cuda")
            self.sets.append(d)

    def launch(self, name, d):
        return row_call(self.ops, name, d, self.cos, self.sin, d.codes, d.scales, d.kc, d.vc)


def row_call(ops, name, d, cos, sin, codes, scales, kc, vc):
    """One call of row `name` on the inputs d (updated in place where the row works in place)."""
    n = d.x.shape[0]
    q = d.qkv[:, :NQ * HD].view(n, NQ, HD)
    k = d.qkv[:, NQ * HD:(NQ + NKV) * HD].view(n, NKV, HD)
    v = d.qkv[:, (NQ + NKV) * HD:].view(n, NKV, HD)
    if name == "rmsnorm_quantize":
        ops.rmsnorm_quantize(d.x, d.w, eps=EPS, gs=64, out_q=codes, out_s=scales)
    elif name == "add_rmsnorm_quantize":
        ops.add_rmsnorm_quantize(d.x, d.add, d.w, eps=EPS, gs=64, out_q=codes, out_s=scales)
    elif name == "kv_pack_f16_kv":
        ops.kv_pack_f16_kv(d.qkv[:, NQ * HD:(NQ + NKV) * HD], d.qkv[:, (NQ + NKV) * HD:], k_out=kc, v_out=vc)
    elif name == "qkv_rope_stage":
        ops.qkv_rope_stage(q, k, v, cos, sin, positions=d.positions, eps=EPS, q_norm_weight=d.q_w,
                           k_norm_weight=d.k_w, k_cache=kc.view(n, NKV, HD), v_cache=vc.view(n, NKV, HD),
                           keep_k_f32=False, keep_v_f32=False)
    elif name == "qkv_bias_rope_only":
        ops.qkv_rope_stage(q, k, v, cos, sin, positions=d.positions, eps=EPS, q_bias=d.bias[:NQ * HD],
                           k_bias=d.bias[NQ * HD:(NQ + NKV) * HD], v_bias=d.bias[(NQ + NKV) * HD:])
    elif name == "add_inplace":
        ops.add_inplace(d.x, d.add)
    else:
        raise ValueError(name)


class ChainArgs(ctypes.Structure):
    """orc_chain_args (oracle/v7_oracle.h): shapes, eps and the host buffers of one chain sample."""
    _fields_ = [(n, ctypes.c_int) for n in
                ("n_tokens", "dim", "n_q_heads", "n_kv_heads", "head_dim", "rope_max_dim", "hidden", "gs")] + [
        ("eps", ctypes.c_float)] + [(n, ctypes.c_void_p) for n in
                                    ("ids", "positions", "table_q", "table_s", "emb_out", "residual", "add",
                                     "w_norm", "normed", "q", "k", "q_w", "k_w", "cos_table", "sin_table",
                                     "gate", "up", "act", "codes", "scales")]


class RowsArgs(ctypes.Structure):
    """orc_rows_args (oracle/v7_oracle.h): the kind, shapes, eps and host buffers of one widened row."""
    _fields_ = [(n, ctypes.c_int) for n in
                ("kind", "n_tokens", "dim", "gs", "n_q_heads", "n_kv_heads", "head_dim", "rope_max_dim")] + [
        ("eps", ctypes.c_float), ("x", ctypes.c_void_p), ("add", ctypes.c_void_p), ("weight", ctypes.c_void_p),
        ("codes", ctypes.c_void_p), ("scales", ctypes.c_void_p), ("qkv", ctypes.c_void_p),
        ("qkv_stride", ctypes.c_longlong)] + [(n, ctypes.c_void_p) for n in
                                              ("q_w", "k_w", "bias", "cos_table", "sin_table", "positions",
                                               "k_cache", "v_cache")]


def rows_leg(torch, ops, chain, L, cores, seconds):
    """The widened rows on the host: the restatement driven per token row over `cores` threads
    (orc_rows_bench, oracle/v7_oracle_rows.c) over all T tokens, and the GPU's outputs of the same inputs
    compared bit for bit (codes, scales, updated rows, cache rows)."""
    import numpy as np

    hostc = lambda t: np.ascontiguousarray(t.detach().cpu().numpy())  # noqa: E731
    L.orc_rows_bench.restype = ctypes.c_double
    L.orc_rows_bench.argtypes = [ctypes.POINTER(RowsArgs), ctypes.c_int, ctypes.c_int, ctypes.c_int]
    src = RowData(torch, T, 7, "cuda")
    h = {k: hostc(getattr(src, k)) for k in ("x", "add", "w", "qkv", "bias", "q_w", "k_w", "positions")}
    cos_t, sin_t = hostc(chain.cos), hostc(chain.sin)
    out = {}
    # the buffers a row touches, per copy: the repetitions cycle through enough copies to span 1.5 GB, more
    # than the host's caches hold
    touched = {"rmsnorm_quantize": ("x", "codes"), "add_rmsnorm_quantize": ("x", "add", "codes"),
               "kv_pack_f16_kv": ("qkv", "kc", "vc"), "qkv_rope_stage": ("qkv", "kc", "vc"),
               "qkv_bias_rope_only": ("qkv",), "add_inplace": ("x", "add")}
    for name, kind in ROW_KINDS.items():
        def copy_set():  # fresh copies of what the row reads or writes; the rest is shared
            b = {k: (v.copy() if k in touched[name] else v) for k, v in h.items()}
            b["codes"] = np.zeros((T, DIM), np.int8)
            b["scales"] = np.zeros((T, DIM // 64), np.float32)
            b["kc"] = np.zeros((T, KVD), np.uint16)
            b["vc"] = np.zeros((T, KVD), np.uint16)
            return b

        def args_of(b):
            p = lambda a: a.ctypes.data  # noqa: E731
            return RowsArgs(kind, T, DIM, 64, NQ, NKV, HD, HD // 2, EPS, p(b["x"]), p(b["add"]), p(b["w"]),
                            p(b["codes"]), p(b["scales"]), p(b["qkv"]), QKV, p(b["q_w"]), p(b["k_w"]), p(b["bias"]),
                            p(cos_t), p(sin_t), p(b["positions"]), p(b["kc"]), p(b["vc"]))

        b = copy_set()
        a = args_of(b)
        L.orc_rows_bench(ctypes.byref(a), 1, cores, 1)
        # the GPU on the same inputs
        d = RowData.__new__(RowData)
        for k in ("x", "add", "w", "qkv", "bias", "q_w", "k_w", "positions"):
            setattr(d, k, getattr(src, k).clone())
        codes = torch.zeros((T, DIM), dtype=torch.int8, device="cuda")
        scales = torch.zeros((T, DIM // 64), dtype=torch.float32, device="cuda")
        kc = torch.zeros((T, KVD), dtype=torch.float16, device="cuda")
        vc = torch.zeros((T, KVD), dtype=torch.float16, device="cuda")
        row_call(ops, name, d, chain.cos, chain.sin, codes, scales, kc, vc)
        torch.cuda.synchronize()
        if name in ("rmsnorm_quantize", "add_rmsnorm_quantize"):
            same = np.array_equal(hostc(codes), b["codes"]) and np.array_equal(hostc(scales), b["scales"])
            same = same and np.array_equal(hostc(d.x), b["x"])
        elif name == "add_inplace":
            same = np.array_equal(hostc(d.x), b["x"])
        elif name == "kv_pack_f16_kv":
            same = np.array_equal(hostc(kc).view(np.uint16), b["kc"]) and np.array_equal(hostc(vc).view(np.uint16),
                                                                                          b["vc"])
        elif name == "qkv_rope_stage":
            same = (np.array_equal(hostc(d.qkv)[:, :NQ * HD], b["qkv"][:, :NQ * HD])
                    and np.array_equal(hostc(kc).view(np.uint16), b["kc"])
                    and np.array_equal(hostc(vc).view(np.uint16), b["vc"]))
        else:
            same = np.array_equal(hostc(d.qkv).view(np.uint32), b["qkv"].view(np.uint32))
        del d, codes, scales, kc, vc
        per_set = sum(b[k].nbytes for k in touched[name])
        sets = [b] + [copy_set() for _ in range(max(1, -(-1_500_000_000 // per_set)) - 1)]
        arr = (RowsArgs * len(sets))(*[args_of(x) for x in sets])
        L.orc_rows_bench(arr, len(sets), cores, len(sets))  # one warm pass over every copy
        # timing: rounds of whole passes over the copies until `seconds` of work have been timed
        secs, reps, chunk = 0.0, 0, len(sets)
        while secs < seconds:
            t = L.orc_rows_bench(arr, len(sets), cores, chunk)
            secs += t
            reps += chunk
            chunk = len(sets) * max(1, min(4 * chunk // len(sets),
                                           int((seconds - secs) / max(t / chunk, 1e-6)) // len(sets) + 1))
        out[name] = {"value": round(ROW_BYTES[name] * reps / secs / 1e9, 3), "unit": "GB/s", "cores": cores,
                     "kind": "port", "form": ROW_FORMS[name], "gpu_bit_exact": bool(same),
                     "sample": f"all {T} tokens, per-row calls, {reps} repetitions in {secs:.1f} s cycling "
                               f"through {len(sets)} copies of the buffers ({len(sets) * per_set / 1e9:.1f} GB)"}
        del sets, arr, b
    return out


def cpu_baseline(torch, ops, chain, args):
    """Times the AVX2 restatement of the reference kernels (oracle/, "port") on a sample of the workload and
    checks the GPU chain bit for bit on the same sample."""
    import numpy as np

    from oracle import oracle as O

    L = O.lib()
    S = min(args.cpu_tokens, T)
    hostc = lambda t: np.ascontiguousarray(t.detach().cpu().numpy())  # noqa: E731
    ids = hostc(chain.ids[:S])
    table_q = hostc(chain.table_q)
    table_s = hostc(chain.table_s)
    residual0 = hostc(chain.residual[:S])
    add = hostc(chain.add[:S])
    w_norm = hostc(chain.w_norm)
    qkv0 = hostc(chain.qkv[:S])
    q_w, k_w = hostc(chain.q_w), hostc(chain.k_w)
    cos_t, sin_t = hostc(chain.cos), hostc(chain.sin)
    positions = np.arange(S, dtype=np.int32)
    gate = hostc(chain.gate[:S])
    up = hostc(chain.up[:S])

    Args = ChainArgs

    def make_args(n, residual, q, k, eps=EPS):
        out = dict(emb=np.empty((S, DIM), np.float32), normed=np.empty((S, DIM), np.float32),
                   act=np.empty((S, HIDDEN), np.float32), codes=np.empty((S, HIDDEN), np.int8),
                   scales=np.empty((S, HIDDEN // GS), np.float32))
        p = lambda a: a.ctypes.data  # noqa: E731
        a = Args(n, DIM, NQ, NKV, HD, HD // 2, HIDDEN, GS, eps, p(ids), p(positions), p(table_q), p(table_s),
                 p(out["emb"]), p(residual), p(add), p(w_norm), p(out["normed"]), p(q), p(k), p(q_w), p(k_w), p(cos_t),
                 p(sin_t), p(gate), p(up), p(out["act"]), p(out["codes"]), p(out["scales"]))
        return a, out

    def run(reps, n_threads, residual, q, k, n=S):
        a, out = make_args(n, residual, q, k)
        L.orc_avx2_chain_bench.restype = ctypes.c_double
        L.orc_avx2_chain_bench.argtypes = [ctypes.POINTER(Args), ctypes.c_int, ctypes.c_int]
        secs = L.orc_avx2_chain_bench(ctypes.byref(a), n_threads, reps)
        return secs, out["emb"], out["normed"], out["codes"], out["scales"]

    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:
        cores = os.cpu_count() or 1
    cores = max(1, min(cores, 64))

    # Parity of the sample: one pass on the CPU, one on the GPU (fresh copies of the same inputs).
    q_h = np.ascontiguousarray(qkv0[:, :NQ * HD])
    k_h = np.ascontiguousarray(qkv0[:, NQ * HD:(NQ + NKV) * HD])
    r_h = residual0.copy()
    _, emb_c, normed_c, codes_c, scales_c = run(1, cores, r_h, q_h, k_h)
    sub = Chain.__new__(Chain)
    sub.n, sub.ops = S, ops
    sub.table_q, sub.table_s, sub.ids = chain.table_q, chain.table_s, chain.ids[:S].clone()
    sub.emb = torch.empty((S, DIM), device="cuda")
    sub.residual, sub.add, sub.w_norm = torch.from_numpy(residual0).cuda(), chain.add[:S].clone(), chain.w_norm
    sub.normed = torch.empty((S, DIM), device="cuda")
    sub.qkv = torch.from_numpy(qkv0).cuda()
    sub.q_w, sub.k_w, sub.cos, sub.sin = chain.q_w, chain.k_w, chain.cos, chain.sin
    sub.positions = torch.arange(S, dtype=torch.int32, device="cuda")
    sub.gate, sub.up = chain.gate[:S].clone(), chain.up[:S].clone()
    sub.codes = torch.empty((S, HIDDEN), dtype=torch.int8, device="cuda")
    sub.scales = torch.empty((S, HIDDEN // GS), device="cuda")
    for _, fn in sub.launches():
        fn()
    torch.cuda.synchronize()
    qkv_g = hostc(sub.qkv)
    match = bool(np.array_equal(hostc(sub.emb), emb_c) and np.array_equal(hostc(sub.residual), r_h)
                 and np.array_equal(hostc(sub.normed), normed_c)
                 and np.array_equal(qkv_g[:, :NQ * HD], q_h) and np.array_equal(qkv_g[:, NQ * HD:(NQ + NKV) * HD], k_h)
                 and np.array_equal(hostc(sub.codes), codes_c) and np.array_equal(hostc(sub.scales), scales_c))

    # Timing: a warm repetition, then rounds of repetitions until `seconds` of work have been timed.
    r_t, q_t, k_t = residual0.copy(), q_h.copy(), k_h.copy()

    def timed(n_threads, n, seconds):
        """(GB/s over all timed rounds, repetitions, seconds, GB/s of the fastest round of at least 0.5 s)."""
        run(1, n_threads, r_t, q_t, k_t, n)
        per_byte = sum(BYTES.values()) * n / T / 1e9
        secs, reps, chunk, best = 0.0, 0, 1, 0.0
        while secs < seconds:
            t, *_ = run(chunk, n_threads, r_t, q_t, k_t, n)
            secs += t
            reps += chunk
            if t >= 0.5:
                best = max(best, per_byte * chunk / t)
            per_rep = max(t / chunk, 1e-6)
            chunk = max(1, min(chunk * 4, int((seconds - secs) / per_rep) + 1))
        return per_byte * reps / secs, reps, secs, best

    gbs, reps, secs, best = timed(cores, S, args.cpu_seconds)
    # One host thread, as the reference engine runs these kernels on its caller thread, over a quarter of the
    # sample (the same rows, still beyond the host caches) for a quarter of the time.
    n1 = max(1, S // 4)
    gbs1, reps1, secs1, _ = timed(1, n1, args.cpu_seconds / 4)
    rows = None if args.no_rows else rows_leg(torch, ops, chain, L, cores, max(0.5, args.cpu_seconds / 10))
    ref_so = os.environ.get("V7_REF_SO")
    reference = None
    if ref_so:
        reference = reference_leg(L, Args, make_args, residual0, q_h, k_h, S, cores, ref_so,
                                  float(os.environ.get("V7_REF_EPS", "0")), args.cpu_seconds)
    return {
        "value": round(gbs, 3), "unit": "GB/s", "cores": cores, "kind": "port",
        "sample": f"{S} of the {T} tokens of the same chain (same shapes; working set larger than the host "
                  f"caches; per-row calls as the reference engine makes them), {reps} repetitions in {secs:.1f} s, "
                  f"row-parallel over {cores} host threads; "
                  f"AVX2 restatement of the NASM kernels (oracle/v7_oracle_avx2.c), not the reference binary",
        # the host's other load moves the average between runs; the fastest round bounds what the host can do
        "best_round_value": round(best, 3) if best else None,
        "single_thread": {"value": round(gbs1, 3), "unit": "GB/s", "cores": 1,
                          "sample": f"{n1} tokens, {reps1} repetitions in {secs1:.1f} s"},
        "cpu_model": cpu_model(),
        "gpu_sample_bit_exact": match,
        **({"rows": rows} if rows is not None else {}),
        **({"reference": reference} if reference is not None else {}),
    }


def reference_leg(L, Args, make_args, residual0, q0, k0, S, cores, path, eps, seconds):
    """The reference library itself (a libv7_threading.so built by its own Makefile, named by V7_REF_SO) on
    the two kernels of the chain it exports, v7s_fused_add_rmsnorm and v7s_rmsnorm_rope_heads
    (src/v7_threading.def, src/v7_lib.h:272-273), timed per token row over the same sample and threads as
    the restatement, whose same two kernels are timed beside it.  The library's norm kernels read eps from
    its g_rms_eps global, 0 unless its database init ran: V7_REF_EPS names the value it holds, and the
    restatement computes with it, so the two outputs are compared bit for bit."""
    import numpy as np

    L.orc_ref_open.restype = ctypes.c_int
    L.orc_ref_open.argtypes = [ctypes.c_char_p]
    L.orc_ref_error.restype = ctypes.c_char_p
    L.orc_k23_bench.restype = ctypes.c_double
    L.orc_k23_bench.argtypes = [ctypes.POINTER(Args), ctypes.c_int, ctypes.c_int, ctypes.c_int]
    rc = L.orc_ref_open(path.encode())
    if rc != 0:
        return {"so": path, "error": L.orc_ref_error().decode(errors="replace")}
    try:
        outs = []
        for use_ref in (1, 0):
            r, q, k = residual0.copy(), q0.copy(), k0.copy()
            a, out = make_args(S, r, q, k, eps)
            L.orc_k23_bench(ctypes.byref(a), cores, 1, use_ref)
            outs.append((r, q, k, out["normed"]))
        same = all(np.array_equal(x.view(np.uint32), y.view(np.uint32)) for x, y in zip(*outs))
        k23_bytes = (BYTES["fused_add_rmsnorm"] + BYTES["qk_rmsnorm_rope"]) * S / T
        res = {}
        for name, use_ref in (("reference", 1), ("port", 0)):
            r, q, k = residual0.copy(), q0.copy(), k0.copy()
            a, _ = make_args(S, r, q, k, eps)
            L.orc_k23_bench(ctypes.byref(a), cores, 1, use_ref)
            secs, reps, chunk = 0.0, 0, 1
            while secs < seconds / 2:
                t = L.orc_k23_bench(ctypes.byref(a), cores, chunk, use_ref)
                secs += t
                reps += chunk
                chunk = max(1, min(chunk * 4, int((seconds / 2 - secs) / max(t / chunk, 1e-6)) + 1))
            res[name] = (k23_bytes * reps / secs / 1e9, reps, secs)
    finally:
        L.orc_ref_close()
    return {
        "so": path, "kernels": ["v7s_fused_add_rmsnorm", "v7s_rmsnorm_rope_heads"], "eps": eps,
        "value": round(res["reference"][0], 3), "unit": "GB/s", "cores": cores,
        "port_same_kernels": round(res["port"][0], 3),
        "bit_exact_vs_port": bool(same),
        "sample": f"add+RMSNorm and Q/K RMSNorm+RoPE of {S} tokens per row, {res['reference'][1]} repetitions "
                  f"in {res['reference'][2]:.1f} s",
    }


class HipEvents:
    """Timing events of the HIP runtime, created with hipEventDisableSystemFence (0x20000000)."""

    def __init__(self):
        self.ct = ctypes
        self.hip = ctypes.CDLL("libamdhip64.so")
        self.hip.hipEventCreateWithFlags.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_uint]
        self.hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.hip.hipEventDestroy.argtypes = [ctypes.c_void_p]
        self.hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self.made = []

    def record(self, e, stream):
        rc = self.hip.hipEventRecord(e, ctypes.c_void_p(stream))
        if rc != 0:
            raise RuntimeError(f"hipEventRecord failed ({rc})")

    def create(self):
        e = self.ct.c_void_p()
        rc = self.hip.hipEventCreateWithFlags(self.ct.byref(e), 0x20000000)
        if rc != 0:
            raise RuntimeError(f"hipEventCreateWithFlags failed ({rc})")
        self.made.append(e)
        return e

    def elapsed_ms(self, a, b):
        f = self.ct.c_float()
        rc = self.hip.hipEventElapsedTime(self.ct.byref(f), a, b)
        if rc != 0:
            raise RuntimeError(f"hipEventElapsedTime failed ({rc})")
        return f.value

    def __del__(self):
        for e in getattr(self, "made", []):
            self.hip.hipEventDestroy(e)


def cpu_model():
    """The first CPU's model name with its family, model and stepping numbers (a virtual machine's model name
    can be as short as "AMD EPYC"; the numbers still name the core generation: family 25 is Zen 3/4, 26 Zen 5)."""
    fields = {}
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if not line.strip():
                    break
                key, _, value = line.partition(":")
                fields[key.strip()] = value.strip()
    except OSError:
        return None
    name = fields.get("model name")
    ids = [f"{k} {fields[k]}" for k in ("cpu family", "model", "stepping") if k in fields]
    if name and ids:
        return f"{name} ({', '.join(ids)})"
    return name


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: the fused per-layer kernels are row-independent and this build "
              "runs on a single MI355X; multi-GPU runs are not supported (use --gpus 1).", file=sys.stderr)
        sys.exit(2)

    import torch

    from v7multiplikator_amd import _lib, ops

    _lib.load()
    torch.cuda.set_device(0)
    chain = Chain(torch, ops, args.seed)
    torch.cuda.synchronize()

    cpu = None
    if not args.no_cpu:
        cpu = cpu_baseline(torch, ops, chain, args)

    launches = chain.launches()
    names = [n for n, _ in launches]
    dom = names.index(DOMINANT)
    if args.copy_probe:
        # A plain copy of a known size (1 GiB read + 1 GiB written) in the same process: under
        # `rocprofv3 --pmc FETCH_SIZE` / `WRITE_SIZE` it gives the counters' scale factor.
        src = torch.empty(1 << 28, dtype=torch.float32, device="cuda").uniform_()
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst
    for _ in range(args.warmup):
        for _, fn in launches:
            fn()
    torch.cuda.synchronize()

    # Timed region: K chain steps back to back.  HIP events on the launch stream (torch's current
    # stream, which the library binds to) time the dominant kernel of every step.
    # v7g_time_next_call hands them to that kernel's launch, so no record call sits between the
    # kernels, and they are created without the system-scope fence, whose cache write-back would
    # otherwise land inside the measured interval and slow the next kernel.
    lib = _lib.load()
    hip = HipEvents()
    ev = [(hip.create(), hip.create()) for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s in range(args.steps):
        for i, (_, fn) in enumerate(launches):
            if i == dom:
                lib.v7g_time_next_call(ev[s][0], ev[s][1])
            fn()
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    dom_ms = sum(hip.elapsed_ms(a, b) for a, b in ev) / args.steps

    # Per-kernel pass (after the timed region, not part of `value`): the same K steps with every
    # kernel timed the same way, for the per-kernel breakdown.
    evk = [[(hip.create(), hip.create()) for _ in launches] for _ in range(args.steps)]
    for s in range(args.steps):
        for (_, fn), (a, b) in zip(launches, evk[s]):
            lib.v7g_time_next_call(a, b)
            fn()
    torch.cuda.synchronize()

    # The widened rows at the same shapes (after the timed region, not part of `value`): each row's calls,
    # rotating through ROW_SETS buffer sets, captured in a HIP graph and replayed between one pair of events, so that
    # neither per-call event markers nor the host's time per call (longer than the 18 us K/V pack) sit
    # between the kernels.
    rows_out = None if args.no_rows else {}
    rows = None if args.no_rows else Rows(torch, ops, chain, args.seed)
    row_reps = max(4, min(args.steps, 20))
    for name in (ROW_BYTES if rows is not None else ()):
        for d in rows.sets:
            rows.launch(name, d)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        try:
            with torch.cuda.graph(graph):
                for i in range(row_reps):
                    rows.launch(name, rows.sets[i % len(rows.sets)])
        finally:
            # the library binds each host thread to the stream of its last call: back to the current stream
            lib.v7g_set_stream(ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
        graph.replay()
        torch.cuda.synchronize()
        e0, e1 = hip.create(), hip.create()
        stream = torch.cuda.current_stream().cuda_stream
        hip.record(e0, stream)
        graph.replay()
        hip.record(e1, stream)
        torch.cuda.synchronize()
        ms = hip.elapsed_ms(e0, e1) / row_reps
        del graph
        gbs = ROW_BYTES[name] / (ms * 1e-3) / 1e9
        rows_out[name] = {"shape": ROW_SHAPES[name], "bytes": ROW_BYTES[name], "us": round(ms * 1e3, 2),
                          "GB/s": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4)}
    del rows

    kern = {}
    for i, (name, _) in enumerate(launches):
        ms = sum(hip.elapsed_ms(*evk[s][i]) for s in range(args.steps)) / args.steps
        gbs = BYTES[name] / (ms * 1e-3) / 1e9
        kern[name] = {"bytes": BYTES[name], "us": round(ms * 1e3, 2), "GB/s": round(gbs, 1),
                      "frac": round(gbs / HBM_PEAK_GBS, 4)}
    total_bytes = sum(BYTES.values())
    value = total_bytes * args.steps / wall / 1e9
    dom_gbs = BYTES[DOMINANT] / (dom_ms * 1e-3) / 1e9

    traffic = None
    tpath = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get(DOMINANT, {}).get("hbm_bytes_per_launch")

    line = {
        "metric": "HBM GB/s & % of 8 TB/s peak: fused add+RMSNorm, RMSNorm+RoPE, SwiGLU-Q8",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded device generator, distributions of the benchmark configurations)",
        "config": {"workload": "Qwen3-8B per-layer elementwise chain, T=8192: Q8 embedding gather (151936x4096), "
                               "add+RMSNorm d=4096, RMSNorm+RoPE 32Q/8KV hd128, SwiGLU->Q8 I=12288 GS=32",
                   "tokens": T, "seed": args.seed, "chain_bytes_per_step": total_bytes, "hbm_fraction_of_peak": round(
                       value / HBM_PEAK_GBS, 4)},
        "roofline": {"bound": "hbm", "kernel": DOMINANT, "achieved": round(dom_gbs, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(dom_gbs / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "us_per_launch": round(dom_ms * 1e3, 2), "algorithmic_bytes": BYTES[DOMINANT]},
        "kernels": kern,
        **({"rows": rows_out} if rows_out is not None else {}),
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
