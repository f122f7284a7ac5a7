"""The C ABI of libv7g.so without a GPU: exports, argument validation, error reporting (CPU only).

Every entry point declared in include/v7g_lib.h must be exported; the batched
entries must reject contract violations with the documented code before any
HIP call, and the drop-in (reference-signature) entries must record them in
the sticky error instead of aborting the host (the reference's FATAL path,
src/asm/v7_core.inc:291-299, has no place in a GPU library).
"""
from __future__ import annotations

import ctypes
import os
import re
import subprocess

import pytest

from v7multiplikator_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "v7g_lib.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = set()
    for m in re.finditer(r"^\s*(?:V7_ABI\s+)?(?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\s*\**\s*([a-z][a-z0-9_]*)\s*\(",
                         text, flags=re.M):
        names.add(m.group(1))
    return sorted(n for n in names if n.startswith(("v7g_", "v7s_", "v7d_")))


@pytest.fixture(scope="module")
def L():
    return _lib.load()


def test_header_declares_the_drop_in_and_batched_entries():
    names = declared_functions()
    for n in ("v7s_fused_add_rmsnorm", "v7s_rmsnorm_rope_heads", "v7d_quantize", "v7s_embedding_row",
              "v7s_swiglu_row", "v7s_swiglu_quantize_row", "v7s_rope_init", "v7g_fused_add_rmsnorm",
              "v7g_rmsnorm_rope_heads", "v7g_qk_rmsnorm_rope", "v7g_swiglu_f32", "v7g_swiglu_q8",
              "v7g_quantize_q8", "v7g_embedding_gather_q8"):
        assert n in names, n


def test_library_exports_every_declared_symbol(L):
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    missing = [n for n in declared_functions() if n not in exported]
    assert not missing, missing
    for n in declared_functions():
        assert getattr(L, n) is not None


def test_library_exports_only_the_c_abi():
    """The kernels and C++ launchers are internal: every exported function is a declared C entry."""
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = sorted(line.split()[-1] for line in out.splitlines() if " T " in line)
    assert exported == declared_functions()


def test_python_binding_covers_the_plain_c_entries():
    plain = [n for n in declared_functions() if n.startswith("v7g_")]
    assert sorted(plain) == sorted(_lib.SIGNATURES)
    drop_in = [n for n in declared_functions() if not n.startswith("v7g_")]
    assert sorted(drop_in) == sorted(_lib.DROP_IN)


def test_error_strings(L):
    for code in range(0, 8):
        assert _lib.error_string(code) not in ("", "unknown error")
    assert _lib.error_string(99) == "unknown error"


def test_eps_global_roundtrip(L):
    old = L.v7g_get_rms_eps()
    try:
        L.v7g_set_rms_eps(1e-5)
        assert abs(L.v7g_get_rms_eps() - 1e-5) < 1e-12
    finally:
        L.v7g_set_rms_eps(old)


def test_rope_config_roundtrip_and_rejects(L):
    """v7g_set_rope_config (the stand-in for the model DB's __sys_rope_* keys that v7s_rope_init reads) keeps
    what it is given, refuses what the table builder cannot use without touching the stored configuration, and
    v7g_clear_rope_config forgets it.  No GPU call is made."""
    c_int, c_f = ctypes.c_int, ctypes.c_float
    out = [c_int(), c_f(), c_f(), c_f(), c_f(), c_int()]
    get = lambda: L.v7g_get_rope_config(*(ctypes.byref(v) for v in out))  # noqa: E731
    L.v7g_clear_rope_config()
    try:
        assert get() == 0
        assert L.v7g_set_rope_config(1, c_f(500000.0), c_f(8.0), c_f(1.0), c_f(4.0), 8192) == 0
        assert get() == 1
        assert [v.value for v in out] == [1, 500000.0, 8.0, 1.0, 4.0, 8192]
        bad = [(2, 1e4, 0, 0, 0, 0), (-1, 1e4, 0, 0, 0, 0), (0, 0.0, 0, 0, 0, 0), (0, -1e4, 0, 0, 0, 0),
               (0, float("inf"), 0, 0, 0, 0), (0, float("nan"), 0, 0, 0, 0), (1, 1e4, 0.0, 1.0, 4.0, 8192),
               (1, 1e4, 8.0, 4.0, 4.0, 8192), (1, 1e4, 8.0, 0.0, 4.0, 8192), (1, 1e4, 8.0, 1.0, 4.0, 0)]
        for t, b, f, lo, hi, op in bad:
            rc, err = _sticky(L, L.v7g_set_rope_config, t, c_f(b), c_f(f), c_f(lo), c_f(hi), op)
            assert rc == 2 and err == 2, (t, b, f, lo, hi, op)
            assert get() == 1 and out[0].value == 1 and out[1].value == 500000.0
        # type 0 keeps only the base: the Llama 3 fields read back as zero
        assert L.v7g_set_rope_config(0, c_f(1e6), c_f(8.0), c_f(1.0), c_f(4.0), 8192) == 0
        assert get() == 1 and [v.value for v in out] == [0, 1e6, 0.0, 0.0, 0.0, 0]
        assert L.v7g_get_rope_config(None, None, None, None, None, None) == 1
        L.v7g_clear_rope_config()
        assert get() == 0
    finally:
        L.v7g_clear_rope_config()
        L.v7g_clear_last_error()


def _sticky(L, fn, *args):
    L.v7g_clear_last_error()
    rc = fn(*args)
    return rc, L.v7g_get_last_error()


FAKE = 0x10000  # a 16-byte aligned non-null address; never dereferenced: validation fails first


@pytest.mark.parametrize("rows,dim,want", [(1, 7, 2), (1, 0, 2), (-1, 64, 2), (1, 16392, 2)])
def test_fused_add_rmsnorm_rejects_shapes(L, rows, dim, want):
    rc, err = _sticky(L, L.v7g_fused_add_rmsnorm, FAKE, FAKE, FAKE, FAKE, rows, dim, 1e-6)
    assert rc == want and err == want


def test_fused_add_rmsnorm_rejects_null_and_misaligned(L):
    assert _sticky(L, L.v7g_fused_add_rmsnorm, None, FAKE, FAKE, FAKE, 2, 64, 1e-6) == (1, 1)
    assert _sticky(L, L.v7g_fused_add_rmsnorm, FAKE + 4, FAKE, FAKE, FAKE, 2, 64, 1e-6) == (3, 3)
    # rows == 0 touches nothing: OK even with NULL pointers
    assert _sticky(L, L.v7g_fused_add_rmsnorm, None, None, None, None, 0, 64, 1e-6) == (0, 0)


@pytest.mark.parametrize("hd", [32, 48, 544, 100])
def test_rope_rejects_head_dims(L, hd):
    rc, err = _sticky(L, L.v7g_rmsnorm_rope_heads, FAKE, 4, 8 * hd, 8, hd, FAKE, FAKE, FAKE, None, 0, hd // 2,
                      16, 1e-6)
    assert rc == 2 and err == 2


def test_rope_rejects_short_table_rows_and_stride(L):
    # rope_max_dim < head_dim/2
    assert _sticky(L, L.v7g_rmsnorm_rope_heads, FAKE, 4, 1024, 8, 128, FAKE, FAKE, FAKE, None, 0, 32, 16,
                   1e-6)[0] == 2
    # token stride shorter than the heads of one token
    assert _sticky(L, L.v7g_rmsnorm_rope_heads, FAKE, 4, 512, 8, 128, FAKE, FAKE, FAKE, None, 0, 64, 16,
                   1e-6)[0] == 2
    # misaligned positions
    assert _sticky(L, L.v7g_rmsnorm_rope_heads, FAKE, 4, 1024, 8, 128, FAKE, FAKE, FAKE, FAKE + 2, 0, 64, 16,
                   1e-6)[0] == 3
    # qk form: k side checked too
    assert _sticky(L, L.v7g_qk_rmsnorm_rope, FAKE, 4096, 32, FAKE, None, 1024, 8, FAKE, 4, 128, FAKE, FAKE, None,
                   0, 64, 16, 1e-6)[0] == 1


@pytest.mark.skipif("__import__('torch').cuda.is_available()",
                    reason="a missed check would launch on the fake pointers; run where no GPU is present")
def test_rope_head_count_sums_cannot_overflow(L):
    """Q + K (+ V) head counts add in 64 bits: 2^30 + 2^30 heads per token is rejected, not wrapped negative."""
    assert _sticky(L, L.v7g_qk_rmsnorm_rope, FAKE, 4096, 1 << 30, FAKE, FAKE, 1024, 1 << 30, FAKE, 1, 128, FAKE,
                   FAKE, None, 0, 64, 16, 1e-6) == (2, 2)


def test_quantize_and_swiglu_reject(L):
    assert _sticky(L, L.v7g_quantize_q8, FAKE, FAKE, FAKE, 1, 64, 0)[0] == 2
    assert _sticky(L, L.v7g_quantize_q8, FAKE, FAKE, FAKE, 1, 64, 8192)[0] == 2
    assert _sticky(L, L.v7g_quantize_q8, None, FAKE, FAKE, 1, 64, 64)[0] == 1
    assert _sticky(L, L.v7g_swiglu_q8, FAKE, FAKE, None, FAKE, 1, 64, 32)[0] == 1
    assert _sticky(L, L.v7g_quantize_q8, FAKE, FAKE + 2, FAKE, 1, 64, 64)[0] == 3  # scales 4-byte aligned
    # gs 1 over 2^38 groups would need more than 2^30 blocks on the general path
    assert _sticky(L, L.v7g_quantize_q8, FAKE, FAKE, FAKE, 1 << 20, 1 << 18, 1)[0] == 2
    assert _sticky(L, L.v7g_swiglu_f32, FAKE, FAKE, FAKE, -1)[0] == 2
    assert _sticky(L, L.v7g_swiglu_f32, FAKE, FAKE, FAKE, 1 << 40)[0] == 2  # one float4 per thread: grid bound
    assert _sticky(L, L.v7g_add_inplace, FAKE, FAKE, 1 << 40)[0] == 2
    assert _sticky(L, L.v7g_swiglu_f32, FAKE, FAKE + 8, FAKE, 16)[0] == 3
    assert _sticky(L, L.v7g_swiglu_f32, None, None, None, 0) == (0, 0)


def test_pointer_checks_switch_and_error_string(L):
    """Pointer checks are off by default (no V7G_CHECK_POINTERS in the environment) and switch per process;
    their error code has its own message.  The checks themselves need a device (tests/test_gpu_parity.py)."""
    before = L.v7g_get_pointer_checks()
    try:
        L.v7g_set_pointer_checks(1)
        assert L.v7g_get_pointer_checks() == 1
        L.v7g_set_pointer_checks(0)
        assert L.v7g_get_pointer_checks() == 0
    finally:
        L.v7g_set_pointer_checks(before)
    assert L.v7g_error_string(6) == b"a pointer is not memory the current device can access"


def test_rope_table_builders_reject(L):
    f = ctypes.c_float
    assert _sticky(L, L.v7g_build_rope_tables_llama3, None, FAKE, 16, 128, f(5e5), f(8), f(1), f(4), 8192)[0] == 1
    assert _sticky(L, L.v7g_build_rope_tables_llama3, FAKE, FAKE, 16, 128, f(5e5), f(0), f(1), f(4), 8192)[0] == 2
    assert _sticky(L, L.v7g_build_rope_tables_llama3, FAKE, FAKE, 16, 128, f(5e5), f(8), f(4), f(4), 8192)[0] == 2
    assert _sticky(L, L.v7g_build_rope_tables_llama3, FAKE, FAKE, 16, 128, f(5e5), f(8), f(1), f(4), 0)[0] == 2
    assert _sticky(L, L.v7g_build_rope_tables_llama3, FAKE, FAKE, 0, 128, f(5e5), f(8), f(1), f(4), 8192)[0] == 2
    assert _sticky(L, L.v7g_rope_init_llama3, 127, f(5e5), 16, f(8), f(1), f(4), 8192)[0] == 2
    assert _sticky(L, L.v7g_rope_init_llama3, 128, f(5e5), 16, f(8), f(1), f(0.5), 8192)[0] == 2


def test_kv_pack_kv_rejects(L):
    f = L.v7g_kv_pack_f16_kv
    assert _sticky(L, f, FAKE, 1024, FAKE + (1 << 20), 1024, FAKE + (2 << 20), FAKE + (3 << 20), 6144, 4, 1022)[0] == 2
    assert _sticky(L, f, FAKE, 1020, FAKE + (1 << 20), 1024, FAKE + (2 << 20), FAKE + (3 << 20), 6144, 4, 1024)[0] == 2
    assert _sticky(L, f, FAKE, 1024, FAKE + (1 << 20), 1024, FAKE + (2 << 20), FAKE + (3 << 20), 512, 4, 1024)[0] == 2
    assert _sticky(L, f, FAKE, 1024, None, 1024, FAKE + (2 << 20), FAKE + (3 << 20), 6144, 4, 1024)[0] == 1
    assert _sticky(L, f, FAKE + 4, 1024, FAKE + (1 << 20), 1024, FAKE + (2 << 20), FAKE + (3 << 20), 6144, 4,
                   1024)[0] == 3
    assert _sticky(L, f, FAKE, 1024, FAKE + (1 << 20), 1024, FAKE + (2 << 20) + 8, FAKE + (3 << 20), 6144, 4,
                   1024)[0] == 3
    assert _sticky(L, f, None, 1024, None, 1024, None, None, 6144, 0, 1024) == (0, 0)


def test_embedding_rejects(L):
    assert _sticky(L, L.v7g_embedding_gather_q8, FAKE, FAKE, 4, FAKE, FAKE, 100, 1000)[0] == 2  # dim % 64
    assert _sticky(L, L.v7g_embedding_gather_q8, FAKE, FAKE, 4, FAKE, FAKE, 128, 0)[0] == 2
    assert _sticky(L, L.v7g_embedding_gather_q8, FAKE, None, 4, FAKE, FAKE, 128, 10)[0] == 1
    assert _sticky(L, L.v7g_embedding_gather_q8, FAKE, FAKE, 4, FAKE + 2, FAKE, 128, 10)[0] == 3
    assert _sticky(L, L.v7g_embedding_gather_q8, FAKE + 4, FAKE, 4, FAKE, FAKE, 128, 10)[0] == 3


def test_sticky_error_keeps_the_first_code(L):
    L.v7g_clear_last_error()
    L.v7g_swiglu_f32(FAKE, FAKE, FAKE, -1)
    L.v7g_quantize_q8(None, FAKE, FAKE, 1, 64, 64)
    assert L.v7g_get_last_error() == 2
    L.v7g_clear_last_error()
    assert L.v7g_get_last_error() == 0


def test_rope_table_entry_validation(L):
    assert _sticky(L, L.v7g_rope_init, 127, ctypes.c_float(1e6), 16)[0] == 2
    assert _sticky(L, L.v7g_rope_init, 128, ctypes.c_float(1e6), 131073)[0] == 2
    assert _sticky(L, L.v7g_build_rope_tables, None, FAKE, 16, 128, ctypes.c_float(1e6))[0] == 1
    assert _sticky(L, L.v7g_get_rope_tables, None, None, None, None)[0] == 5


def test_check_raises_and_clears(L):
    L.v7g_clear_last_error()
    rc = L.v7g_swiglu_f32(FAKE, FAKE, FAKE, -1)
    with pytest.raises(_lib.V7GError) as e:
        _lib.check(rc, "swiglu")
    assert e.value.code == 2
    assert L.v7g_get_last_error() == 0


def test_ops_refuse_host_tensors():
    torch = pytest.importorskip("torch")
    from v7multiplikator_amd import ops

    x = torch.zeros(4, 64)
    with pytest.raises(ValueError):
        ops.swiglu(x, x)
    with pytest.raises(ValueError):
        ops.fused_add_rmsnorm(x, x, torch.ones(64))
    with pytest.raises(TypeError):
        ops.quantize_q8(x.double())


def test_stream_query_falls_back_to_the_public_call(monkeypatch):
    """A raw current-stream query that rejects its argument hands over to torch.cuda.current_stream for good."""
    torch = pytest.importorskip("torch")
    from v7multiplikator_amd import ops

    calls = []

    def raw(index):
        calls.append(index)
        raise TypeError("signature changed")

    class Public:
        cuda_stream = 0x5000

    monkeypatch.setattr(ops, "_raw_stream", raw)
    monkeypatch.setattr(torch.cuda, "current_stream", lambda device=None: Public())
    dev = torch.device("cuda", 0)
    assert ops.current_stream_handle(dev) == 0x5000
    assert ops._raw_stream is None
    assert ops.current_stream_handle(dev) == 0x5000
    assert calls == [0]


def test_stream_binding_is_per_host_thread(L):
    """v7g_set_stream binds the calling thread's launch stream; another thread keeps its own."""
    import threading

    seen = {}
    barrier = threading.Barrier(2)

    def worker(name, value):
        L.v7g_set_stream(value)
        barrier.wait()
        seen[name] = L.v7g_get_stream()

    a = threading.Thread(target=worker, args=("a", 0x1000))
    b = threading.Thread(target=worker, args=("b", 0x2000))
    a.start(), b.start()
    a.join(), b.join()
    assert seen == {"a": 0x1000, "b": 0x2000}
    assert L.v7g_get_stream() in (None, 0)  # this thread never set one


def test_bench_refuses_more_than_one_gpu():
    """bench.py measures one GPU; --gpus N > 1 exits with status 2 and says so, before touching a device."""
    import subprocess
    import sys

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    r = subprocess.run([sys.executable, os.path.join(root, "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr
