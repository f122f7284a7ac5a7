"""The reference-binary baseline leg (oracle/v7_ref_leg.c, bench.reference_leg) on the CPU.

The reference library itself needs nasm, which this image lacks, so these tests drive the leg with a test
double (tests/ref_double.c): a library exporting v7s_fused_add_rmsnorm and v7s_rmsnorm_rope_heads with the
reference's names, signatures and ms_abi convention (src/v7_lib.h:272-273), backed by the AVX2
restatement at an eps held in a global.  Matching the restatement bit for bit through the leg pins the
leg's loading, calling convention and argument order; the eps tests show the comparison has teeth.
"""
import ctypes
import os
import subprocess

import numpy as np
import pytest

import bench
from oracle import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(ROOT, "oracle")

S, DIM, NQ, NKV, HD = 24, 256, 4, 2, 64
RMD = HD // 2


@pytest.fixture(scope="module")
def double_so(tmp_path_factory):
    out = tmp_path_factory.mktemp("ref_double") / "libv7_threading_double.so"
    cmd = ["gcc", "-O2", "-mfma", "-shared", "-fPIC", "-o", str(out), os.path.join(ROOT, "tests", "ref_double.c"),
           "-L", ORACLE_DIR, "-loracle", f"-Wl,-rpath,{ORACLE_DIR}"]
    subprocess.run(cmd, check=True, capture_output=True)
    return str(out)


@pytest.fixture(scope="module")
def L():
    lib = O.lib()
    lib.orc_ref_open.restype = ctypes.c_int
    lib.orc_ref_open.argtypes = [ctypes.c_char_p]
    lib.orc_ref_error.restype = ctypes.c_char_p
    lib.orc_k23_bench.restype = ctypes.c_double
    lib.orc_k23_bench.argtypes = [ctypes.POINTER(bench.ChainArgs), ctypes.c_int, ctypes.c_int, ctypes.c_int]
    yield lib
    lib.orc_ref_close()


def _sample(seed=3):
    rng = np.random.default_rng(seed)
    f = lambda *shape: rng.standard_normal(shape).astype(np.float32)  # noqa: E731
    cos_t, sin_t = O.rope_tables(S, HD, 1e6)
    return dict(residual=f(S, DIM), add=f(S, DIM), w_norm=(1 + 0.1 * f(DIM)).astype(np.float32),
                q=f(S, NQ * HD), k=f(S, NKV * HD), q_w=(1 + 0.1 * f(HD)).astype(np.float32),
                k_w=(1 + 0.1 * f(HD)).astype(np.float32), cos=np.ascontiguousarray(cos_t, np.float32),
                sin=np.ascontiguousarray(sin_t, np.float32),
                positions=rng.permutation(S).astype(np.int32))


def _make_args_fn(d):
    """make_args as bench.cpu_baseline defines it, over the sample d (only the fields the leg reads)."""
    keep = []

    def make_args(n, residual, q, k, eps=1e-6):
        out = dict(normed=np.empty((S, DIM), np.float32))
        p = lambda a: a.ctypes.data  # noqa: E731
        a = bench.ChainArgs(n, DIM, NQ, NKV, HD, RMD, 0, 32, eps, None, p(d["positions"]), None, None, None,
                            p(residual), p(d["add"]), p(d["w_norm"]), p(out["normed"]), p(q), p(k), p(d["q_w"]),
                            p(d["k_w"]), p(d["cos"]), p(d["sin"]), None, None, None, None, None)
        keep.append((a, out, residual, q, k))
        return a, out

    return make_args


def _run(L, d, eps, use_ref):
    make_args = _make_args_fn(d)
    r, q, k = d["residual"].copy(), d["q"].copy(), d["k"].copy()
    a, out = make_args(S, r, q, k, eps)
    secs = L.orc_k23_bench(ctypes.byref(a), 3, 1, use_ref)
    assert secs >= 0
    return r, q, k, out["normed"]


def _set_double_eps(so, eps):
    ctypes.c_float.in_dll(ctypes.CDLL(so), "ref_double_eps").value = eps


def bits(a):
    return a.view(np.uint32)


@pytest.mark.parametrize("eps", [0.0, 1e-6])
def test_leg_matches_restatement_through_the_double(L, double_so, eps):
    assert L.orc_ref_open(double_so.encode()) == 0, L.orc_ref_error()
    _set_double_eps(double_so, eps)
    d = _sample()
    ref = _run(L, d, eps, 1)
    port = _run(L, d, eps, 0)
    for x, y in zip(ref, port):
        assert np.array_equal(bits(x), bits(y))
    # the residual was updated in place and the heads rotated: the leg wrote every output
    assert not np.array_equal(ref[0], d["residual"]) and not np.array_equal(ref[1], d["q"])
    assert not np.array_equal(ref[2], d["k"])
    # and against the scalar oracle's rows (fused add+RMSNorm of every token row)
    o_o, r_o = O.fused_add_rmsnorm(d["residual"], d["add"], d["w_norm"], eps)
    assert np.array_equal(bits(ref[3]), bits(o_o)) and np.array_equal(bits(ref[0]), bits(r_o))


def test_leg_detects_an_eps_mismatch(L, double_so):
    assert L.orc_ref_open(double_so.encode()) == 0
    _set_double_eps(double_so, 0.0)
    d = _sample(4)
    ref = _run(L, d, 0.0, 1)
    port = _run(L, d, 1e-3, 0)
    assert not np.array_equal(bits(ref[3]), bits(port[3]))


def test_leg_errors(L):
    assert L.orc_ref_open(b"/nonexistent/libv7_threading.so") == -1
    assert b"failed to load" in L.orc_ref_error()
    # a library without the two exports (the oracle itself)
    assert L.orc_ref_open(os.path.join(ORACLE_DIR, "liboracle.so").encode()) == -2
    assert b"missing required export 'v7s_fused_add_rmsnorm'" in L.orc_ref_error()
    d = _sample()
    a, _ = _make_args_fn(d)(S, d["residual"].copy(), d["q"].copy(), d["k"].copy())
    assert L.orc_k23_bench(ctypes.byref(a), 1, 1, 1) == -1.0  # nothing loaded


def test_bench_reference_leg_end_to_end(L, double_so):
    _set_double_eps(double_so, 0.0)
    d = _sample(5)
    res = bench.reference_leg(L, bench.ChainArgs, _make_args_fn(d), d["residual"], d["q"], d["k"], S, 2, double_so,
                              0.0, 0.2)
    assert res["bit_exact_vs_port"] is True
    assert res["kernels"] == ["v7s_fused_add_rmsnorm", "v7s_rmsnorm_rope_heads"]
    assert res["value"] > 0 and res["port_same_kernels"] > 0 and res["so"] == double_so
    bad = bench.reference_leg(L, bench.ChainArgs, _make_args_fn(d), d["residual"], d["q"], d["k"], S, 2,
                              "/nonexistent/libv7_threading.so", 0.0, 0.2)
    assert "error" in bad and "failed to load" in bad["error"]
