"""Builds libv7g.so for gfx950 with hipcc, in-tree (next to this file).

    python -m v7multiplikator_amd.build

Flags: -O3, -ffp-contract=off (every a*b+c stays two roundings; the kernels
place every fused multiply-add explicitly, as the reference places vfmadd),
-fgpu-flush-denormals-to-zero (f32 denormals flushed on input and output, the
reference's MXCSR FTZ+DAZ),
packed-FP32 instructions disabled (-Xclang -target-feature -Xclang
-packed-fp32-ops), default correctly rounded f32 division and sqrt.
"""
from __future__ import annotations

import glob
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
LIB = os.path.join(PKG, "libv7g.so")
ARCH = os.environ.get("V7G_OFFLOAD_ARCH", "gfx950")

HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-shared", "-ffp-contract=off",
    "-fgpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # The first kernel-argument dwords arrive in SGPRs at wave launch instead of
    # through a scalar load and its wait at the start of every wave (the code
    # keeps a prologue that loads them itself where the firmware does not
    # preload).
    "-mllvm", "-amdgpu-kernarg-preload-count=14",
    "-Wall", "-Wno-unused-function",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def sources():
    return sorted(glob.glob(os.path.join(CSRC, "*.hip")))


# Host-only C++ (x87 RoPE table builder): compiled by g++ and linked into the library.
HOST_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-ffp-contract=off", "-fno-fast-math", "-Wall"]


def host_sources():
    return sorted(glob.glob(os.path.join(CSRC, "*.cpp")))


def build_library(verbose: bool = False) -> str:
    """Compiles every csrc/*.hip (hipcc, gfx950) and the host-only table builder (g++) into libv7g.so;
    returns its path."""
    tmp = LIB + ".tmp"
    objs = []
    for src in host_sources():
        if os.path.basename(src) == "v7g_loadtest.cpp":
            continue
        obj = os.path.join(PKG, os.path.basename(src) + ".o")
        cmd = ["g++", *HOST_FLAGS, "-c", "-o", obj, src]
        if verbose:
            print(" ".join(cmd), flush=True)
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"g++ failed ({res.returncode}):\n{res.stdout}{res.stderr}")
        objs.append(obj)
    exports = os.path.join(CSRC, "v7g_exports.map")
    cmd = [hipcc(), *HIP_FLAGS, "-I", os.path.join(ROOT, "include"), f"-Wl,--version-script={exports}", "-o", tmp,
           *sources(), "-x", "none", *objs]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    for obj in objs:
        os.remove(obj)
    out = "\n".join(l for l in (res.stdout + res.stderr).splitlines() if "packed-fp32-ops" not in l)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{out}")
    if verbose and out.strip():
        print(out)
    os.replace(tmp, LIB)
    return LIB


def build_loadtest(verbose: bool = False) -> str:
    """Builds the C++ harness csrc/v7g_loadtest.cpp (host only, dlopens libv7g.so)."""
    src = os.path.join(CSRC, "v7g_loadtest.cpp")
    exe = os.path.join(PKG, "v7g_loadtest")
    cmd = ["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-I", os.path.join(ROOT, "include"),
           "-I", "/opt/rocm/include", "-D__HIP_PLATFORM_AMD__", "-o", exe, src, "-ldl",
           "-L/opt/rocm/lib", "-lamdhip64", "-Wl,-rpath,/opt/rocm/lib"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"g++ failed ({res.returncode}):\n{res.stdout}{res.stderr}")
    return exe


def build_fp_env_probe(verbose: bool = False) -> str:
    """Test support: tests/fp_env.hip (flush-mode gfx950 arithmetic against SSE under MXCSR FTZ+DAZ), built
    with the library's flags as tests/v7g_fp_env."""
    src = os.path.join(ROOT, "tests", "fp_env.hip")
    exe = os.path.join(ROOT, "tests", "v7g_fp_env")
    cmd = [hipcc(), *[f for f in HIP_FLAGS if f not in ("-shared", "-fPIC")], "-o", exe, src]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        out = "\n".join(l for l in (res.stdout + res.stderr).splitlines() if "packed-fp32-ops" not in l)
        raise RuntimeError(f"hipcc failed ({res.returncode}):\n{out}")
    return exe


def build_test_shim(verbose: bool = False) -> str:
    """Test support: tests/libdropin_shim.so, System V wrappers of the ms_abi drop-in entries."""
    src = os.path.join(ROOT, "tests", "dropin_shim.c")
    out = os.path.join(ROOT, "tests", "libdropin_shim.so")
    cmd = ["gcc", "-O2", "-shared", "-fPIC", "-I", os.path.join(ROOT, "include"), "-o", out, src, "-L", PKG,
           "-lv7g", "-Wl,-rpath,$ORIGIN/../v7multiplikator_amd"]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"gcc failed ({res.returncode}):\n{res.stdout}{res.stderr}")
    return out


if __name__ == "__main__":
    print(build_library(verbose=True))
    if os.path.exists(os.path.join(CSRC, "v7g_loadtest.cpp")):
        print(build_loadtest(verbose=True))
    sys.exit(0)
