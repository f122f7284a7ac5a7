"""The GPU leg of the reference's load tests (tools/b_fused_add_rmsnorm_loadtest.cpp and its siblings):
v7multiplikator_amd/v7g_loadtest.  On the CPU: arguments are checked before the library or the GPU is touched.
On the GPU: every mode family runs, prints the reference harnesses' "Pass:" line and one JSON record per kernel
whose bytes match the shape it names."""
from __future__ import annotations

import json
import os
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "v7multiplikator_amd")
EXE = os.path.join(PKG, "v7g_loadtest")
LIB = os.path.join(PKG, "libv7g.so")

MODES = ["fused_add_rmsnorm", "rmsnorm", "add_inplace", "rmsnorm_rope", "swiglu", "swiglu_q8", "embedding", "rmsnorm_quantize",
         "add_rmsnorm_quantize", "kv_pack", "kv_pack_kv", "qkv_stage", "rope_only", "configs", "next", "models",
         "decode"]


@pytest.fixture(scope="module")
def exe():
    if not os.path.exists(EXE):
        from v7multiplikator_amd import build
        build.build_loadtest()
    return EXE


def run(exe, *args, timeout=120):
    return subprocess.run([exe, *map(str, args)], capture_output=True, text=True, timeout=timeout)


def test_usage_names_every_mode(exe):
    r = run(exe)
    assert r.returncode == 1
    for mode in MODES:
        assert mode in r.stdout, mode


@pytest.mark.parametrize("args", [["bogus"], ["fused_add_rmsnorm", "8"], ["rmsnorm_rope", "8", "2", "1"],
                                  ["swiglu_q8", "0", "64"], ["models", "0"], ["models", "Llama-3-8B"],
                                  ["embedding", "8", "-3", "64"], ["fused_add_rmsnorm", "8", "64", "--iterations",
                                                                   "0"], ["rmsnorm", "8"], ["add_inplace", "0", "64"]])
def test_bad_arguments_print_usage_before_any_gpu_call(exe, args):
    # the library path does not exist: a run that got past the argument check would report the failed dlopen
    r = run(exe, "/nonexistent/libv7g.so", *args)
    assert r.returncode == 1
    assert r.stdout.startswith("usage:"), r.stdout


def test_unknown_model_shape_is_refused(exe):
    r = run(exe, "/nonexistent/libv7g.so", "models", "64", "NoSuchModel")
    assert r.returncode == 1
    assert "no model shape named NoSuchModel" in r.stdout and "Llama-3-8B" in r.stdout


def records(stdout):
    return [json.loads(l) for l in stdout.splitlines() if l.startswith("{")]


@pytest.mark.gpu
def test_models_mode_runs_the_four_kernels(exe):
    r = run(exe, LIB, "models", 256, "TinyLlama-1.1B", "--iterations", 3, "--no-rotate")
    assert r.returncode == 0, r.stdout + r.stderr
    recs = records(r.stdout)
    assert [x["kernel"] for x in recs] == ["embedding_gather_q8", "fused_add_rmsnorm", "qkv_rope_stage", "swiglu_q8"]
    T, dim, nq, nkv, hd, hidden = 256, 2048, 32, 4, 64, 5632
    assert recs[1]["bytes"] == 16 * T * dim + 4 * dim
    assert recs[2]["bytes"] == 2 * T * (nq + nkv) * hd * 4 + 2 * T * (hd // 2) * 4
    assert recs[3]["bytes"] == 2 * T * hidden * 4 + T * hidden + T * (hidden // 32) * 4
    for x in recs:
        assert x["us"] > 0 and 0 < x["frac"] < 1.2, x
    assert r.stdout.count("Pass: ") == 4


@pytest.mark.gpu
@pytest.mark.parametrize("args,kernel", [(["rope_only", 128, 28, 4, 128, 1], "qkv_rope_stage"),
                                         (["rmsnorm_rope", 128, 16, 8, 256], "rmsnorm_rope"),
                                         (["fused_add_rmsnorm", 64, 5120], "fused_add_rmsnorm"),
                                         (["embedding", 64, 1000, 5120], "embedding_gather_q8"),
                                         (["rmsnorm_quantize", 64, 3584, 64], "rmsnorm_quantize"),
                                         (["kv_pack_kv", 64, 1024], "kv_pack_f16_kv"),
                                         (["rmsnorm", 64, 2048], "rmsnorm"),
                                         (["add_inplace", 64, 4096], "add_inplace")])
def test_single_kernel_modes(exe, args, kernel):
    r = run(exe, LIB, *args, "--iterations", 3, "--no-rotate")
    assert r.returncode == 0, r.stdout + r.stderr
    recs = records(r.stdout)
    assert len(recs) == 1 and recs[0]["kernel"] == kernel, recs
    assert recs[0]["us"] > 0 and "cache-resident" in r.stdout


@pytest.mark.gpu
@pytest.mark.parametrize("mode,bytes_per_call", [("rmsnorm", lambda r, d: 8 * r * d + 4 * d),
                                                 ("add_inplace", lambda r, d: 12 * r * d)])
def test_per_row_modes_of_the_adjacent_harnesses(exe, mode, bytes_per_call):
    """The GPU legs of b_rmsnorm_loadtest and b_add_inplace_loadtest: the batched entry and, with --per-row, the
    reference-signature entry once per row; both count each tensor once."""
    rows, dim = 16, 1024
    for extra in ([], ["--per-row"]):
        r = run(exe, LIB, mode, rows, dim, "--iterations", 3, "--no-rotate", *extra)
        assert r.returncode == 0, r.stdout + r.stderr
        recs = records(r.stdout)
        assert len(recs) == 1 and recs[0]["kernel"] == mode, recs
        assert recs[0]["bytes"] == bytes_per_call(rows, dim) and recs[0]["us"] > 0
        assert ("per-row-calls" in recs[0]["shape"]) == bool(extra)


@pytest.mark.gpu
def test_decode_mode_times_eager_and_graph_steps(exe):
    r = run(exe, LIB, "decode", 4, "--iterations", 5)
    assert r.returncode == 0, r.stdout + r.stderr
    recs = records(r.stdout)
    assert len(recs) == 1 and recs[0]["kernel"] == "decode_step" and recs[0]["tokens"] == 4, recs
    for key in ("eager_us", "host_us_per_call", "graph_per_step_us", "graph_all_steps_us"):
        assert recs[0][key] > 0, key
