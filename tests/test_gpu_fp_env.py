"""gfx950 arithmetic in the library's flush mode (f32 denormals flushed on input and output) against x86 SSE
under MXCSR FTZ+DAZ, the reference's mode (src/asm/v7_init.inc:103-108, src/asm/v7_core.inc:301-303):
every operation the kernels use, on 2^20 operand triples at the denormal boundary, must give the same bits
(tests/fp_env.hip, built with the library's flags as tests/v7g_fp_env)."""
from __future__ import annotations

import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

EXE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "v7g_fp_env")


def test_flush_mode_arithmetic_equals_sse_ftz_daz():
    if not os.path.exists(EXE):
        pytest.fail("v7g_fp_env is not built: run __graft_entry__.build()")
    r = subprocess.run([EXE, "--count", str(1 << 20)], capture_output=True, text=True, timeout=120)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    lines = [l for l in r.stdout.splitlines() if "mismatches" in l]
    assert len(lines) == 11 and all(l.split("mismatches ")[1].startswith("0 of") for l in lines), r.stdout
