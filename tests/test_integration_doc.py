"""The loader a v7 host would add (the C block of the repository's integration guide) compiles as C11 against
include/v7g_lib.h and resolves every entry it lists from the built libv7g.so (dlopen/dlsym only: no GPU call is
made)."""
from __future__ import annotations

import os
import re
import shutil
import subprocess
import tempfile

import pytest

from v7multiplikator_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

MAIN = r'''
#include "v7g_load.h"
int main(int argc, char **argv) {
    if (argc < 2) return 2;
    v7g_lib lib;
    if (v7g_load(argv[1], &lib)) return 1;
    printf("loaded\n");
    return 0;
}
'''


def test_integration_loader_compiles_and_resolves():
    if shutil.which("gcc") is None:
        pytest.skip("gcc is needed")
    text = open(os.path.join(ROOT, "INTEGRATION.md")).read()
    blocks = re.findall(r"```c\n(.*?)```", text, flags=re.S)
    assert blocks, "INTEGRATION.md holds no C loader"
    with tempfile.TemporaryDirectory() as d:
        with open(os.path.join(d, "v7g_load.h"), "w") as f:
            f.write(blocks[0])
        with open(os.path.join(d, "main.c"), "w") as f:
            f.write(MAIN)
        exe = os.path.join(d, "loader")
        subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", "-I", os.path.join(ROOT, "include"), "-I", d, "-o", exe,
                        os.path.join(d, "main.c"), "-ldl"], check=True, capture_output=True, text=True)
        r = subprocess.run([exe, _lib.LIB_PATH], capture_output=True, text=True, timeout=60)
        assert r.returncode == 0 and "loaded" in r.stdout, r.stdout + r.stderr
    # every drop-in entry the library exports is one a host can bind through this loader
    resolved = set(re.findall(r"V7G_RESOLVE\((\w+)\)", blocks[0])) - {"name"}
    missing = [n for n in _lib.DROP_IN if n not in resolved]
    assert not missing, missing
