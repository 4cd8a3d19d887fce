"""The HIP execution layer on the GPU (include/cairn/cairn_ops.hpp and cairn_hip_kernels.hpp over cairn_context.hpp), through the scenario
programs of tests/cpp/exec_device.hip: the device half of the execution-context row (the reference's
src/cairn/runtime/cairn_exec.hpp:25-230, cairn_reuse.hpp:1-525, cairn_gpu.hpp:47-126). Each result is checked
against numpy; the integer folds are exact, so any association order the device library picks gives the same
numbers. The same rules on a recording host machine (waits, allocations, growth, tickets) are
tests/test_cpp_surface.py's."""

from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np
import pytest

from cairn_amd import hip

pytestmark = pytest.mark.gpu

LIB = Path(__file__).resolve().parent / "cpp" / "libexec_device.so"


@pytest.fixture(scope="module")
def ex():
    if not LIB.exists():
        pytest.fail(f"{LIB} is not built: run __graft_entry__.build()")
    lib = C.CDLL(str(LIB))
    P = C.c_void_p
    lib.exec_regions.argtypes = [C.c_size_t, P, P, P, P, P, P, P]
    lib.exec_streams.argtypes = [C.c_size_t, P, P, P]
    lib.exec_queue.argtypes = [C.c_size_t, P]
    lib.exec_budget.argtypes = [C.c_size_t, C.c_size_t, P, P, P]
    lib.exec_owners.argtypes = [P, P]
    lib.exec_resident.argtypes = [C.c_size_t, P, P]
    for f in (lib.exec_regions, lib.exec_streams, lib.exec_queue, lib.exec_budget, lib.exec_owners, lib.exec_resident):
        f.restype = C.c_int
    return lib


def ptr(a: np.ndarray) -> int:
    return a.ctypes.data


@pytest.mark.parametrize("n", [1, 1000, 65536 * 4 + 37, (1 << 23) + 12345])
def test_regions_reductions_scans_and_plans(ex, n):
    sums = np.zeros(4, np.int64)
    inc, exc, kept = (np.zeros(n, np.int64) for _ in range(3))
    used = np.zeros(1, np.uint64)
    vec, stencil = np.zeros(n, np.float32), np.zeros(n, np.float32)
    assert ex.exec_regions(n, ptr(sums), ptr(inc), ptr(exc), ptr(kept), ptr(used), ptr(vec), ptr(stencil)) == 0
    x = (np.arange(n) % 97 - 48).astype(np.int64)
    assert sums[0] == 0  # a fresh buffer reads zeros
    assert sums[1] == x.sum()
    assert sums[2] == x.sum() and sums[3] == x.sum()  # both scans' totals
    assert np.array_equal(inc, np.cumsum(x))
    assert np.array_equal(exc, np.concatenate([[0], np.cumsum(x)[:-1]]))
    sel = np.nonzero(x > 0)[0]
    assert int(used[0]) == len(sel) and np.array_equal(kept[: len(sel)], sel)
    v = (0.5 * np.arange(n, dtype=np.float32)).astype(np.float32)
    assert np.array_equal(vec, v)
    pad = np.concatenate([[0.0], v, [0.0]]).astype(np.float32)
    want = (pad[:-2] + pad[1:-1]).astype(np.float32) + pad[2:]
    assert np.array_equal(stencil, want.astype(np.float32))


def test_held_and_enqueued_work(ex):
    n = 4096
    s = hip.Stream()
    out = np.zeros(2 * n, np.int32)
    waited = np.zeros(1, np.int32)
    try:
        assert ex.exec_streams(n, s.handle, ptr(out), ptr(waited)) == 0
    finally:
        s.close()
    i = np.arange(n)
    assert np.array_equal(out[:n], 2 * (i + 1))
    assert np.array_equal(out[n:], 7 * i)


def test_queued_work_follows_its_tickets(ex):
    n = 100_000
    out = np.zeros(n, np.int32)
    assert ex.exec_queue(n, ptr(out)) == 0  # every lane back after the waits
    assert np.array_equal(out, 3 * (np.arange(n) - 5))


def test_a_budget_answers_over_budget_and_changes_nothing(ex):
    answers = np.full(3, -1, np.int32)
    caps = np.zeros(3, np.uint64)
    total = np.zeros(1, np.int64)
    limit, big = 65536, 100_000  # the scan's held prefix alone (800 KB) passes the limit
    assert ex.exec_budget(limit, big, ptr(answers), ptr(caps), ptr(total)) == 0
    assert list(answers) == [0, 1, 0]  # ok, over_budget, ok
    assert 0 < caps[0] <= limit and caps[1] == caps[0] and caps[2] == caps[0]  # no growth past the limit
    assert total[0] == 45


def test_owners_and_zeroing(ex):
    out = np.zeros(16, np.int32)
    b = np.zeros(37, np.uint8)
    assert ex.exec_owners(ptr(out), ptr(b)) == 0  # pinned storage started zeroed
    assert b[0] == 0xFF and b[36] == 0xFF and not b[1:36].any()  # zero() at an odd address, 35 bytes
    if out[0] == -1:
        pytest.skip("the device reports no coherent access to managed memory: the unified owner is not exercised")
    assert np.array_equal(out, np.arange(16) ** 2)


def test_device_resident_results_and_the_scalar_fallback(ex):
    n = 1003
    out = np.zeros(12, np.int64)
    vec = np.zeros(n, np.float32)
    assert ex.exec_resident(n, ptr(out), ptr(vec)) == 0
    assert out[0] == 499500  # reduce_to, read after its ticket's wait
    assert out[1] == 2 * 4950  # reduce_into inside a held run
    assert np.array_equal(out[2:], np.concatenate([[0], np.cumsum(np.arange(9))]))  # scan_into, exclusive
    assert np.array_equal(vec, 3.0 * np.arange(n, dtype=np.float32))  # the scalar lanes, and the empty region left it
