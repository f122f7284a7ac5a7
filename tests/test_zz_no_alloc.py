"""GPU: the non-allocating self-check equals the allocating one, through the C ABI.

v7g_arith_selfcheck_noalloc keeps its four mismatch counters in the library's
static device memory instead of a buffer it allocates.  Two calls in a row --
all four identities, then only identities 0 and 1 (the smaller input: 2^31
patterns each, against 2^32 for identities 2 and 3) -- must give exactly what
v7g_arith_selfcheck gives for the identities they select, leave the other
entries of the caller's array alone, and start from cleared counters each
time (the second call would otherwise add to the first call's counts).
"""
from __future__ import annotations

import ctypes

import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

SENTINEL = 0xDEADBEEF12345678


@pytest.fixture(scope="module")
def L():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a visible MI355X")
    from v7multiplikator_amd import _lib
    return _lib.load()


def _counts(values):
    return (ctypes.c_ulonglong * 4)(*values)


def test_noalloc_selfcheck_equals_the_allocating_entry_twice(L):
    print("entry: v7g_arith_selfcheck, then v7g_arith_selfcheck_noalloc(0xF), (0x3)", flush=True)
    ref = _counts([SENTINEL] * 4)
    assert L.v7g_arith_selfcheck(ref) == 0
    first = _counts([SENTINEL] * 4)
    assert L.v7g_arith_selfcheck_noalloc(first, 0xF) == 0
    assert list(first) == list(ref)
    second = _counts([SENTINEL] * 4)
    assert L.v7g_arith_selfcheck_noalloc(second, 0x3) == 0
    assert list(second[:2]) == list(ref[:2])
    assert list(second[2:]) == [SENTINEL, SENTINEL]
    assert list(ref) == [0, 0, 0, 0]  # a conforming device


def test_noalloc_selfcheck_from_two_host_threads(L):
    """Two host threads call the non-allocating entry on the same device at once, twice each: the entry holds
    a per-device lock from clearing the shared counters until its counts are back, so every call returns the
    allocating entry's counts for the identities it selects."""
    import threading

    print("entry: v7g_arith_selfcheck_noalloc(0x3) from two host threads", flush=True)
    results, errors = [], []

    def worker():
        try:
            for _ in range(2):
                out = _counts([SENTINEL] * 4)
                rc = L.v7g_arith_selfcheck_noalloc(out, 0x3)
                results.append((rc, list(out)))
        except Exception as e:  # noqa: BLE001
            errors.append(e)

    threads = [threading.Thread(target=worker) for _ in range(2)]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=120)
    assert not errors and len(results) == 4
    for rc, out in results:
        assert rc == 0 and out == [0, 0, SENTINEL, SENTINEL]


def test_noalloc_selfcheck_refuses_more_than_four_identities(L):
    out = _counts([SENTINEL] * 4)
    L.v7g_clear_last_error()
    assert L.v7g_arith_selfcheck_noalloc(out, 0x10) == 2
    assert L.v7g_arith_selfcheck_noalloc(out, 0) == 2
    assert L.v7g_arith_selfcheck_noalloc(None, 0xF) == 1
    L.v7g_clear_last_error()
    assert list(out) == [SENTINEL] * 4
