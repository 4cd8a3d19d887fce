"""The multiply's CAIRN entries on the GPU: cf_mma_<fmt>_device (checked, synchronous on the calling thread's
execution context: cr::tensor::launch<A>(cr::gpu::here(), ...) on the HIP machine), cq_mma_<fmt>_device (the same
work queued on the caller's stream, never waited for) and cairn_gemm_device_stream (the thread's device work bound to
a caller-owned stream), called through ctypes on device views, as tests/soundness/test_tensor.py:31-36,58-62 binds
the entries CAIRN's header generator emits (src/cairn/compiler/lower/header.py:215-249,283-313).

- The reference's device check (tests/soundness/test_tensor.py:183-222): its seven shapes and its generator
  ((e + seed) * 2654435761 % 61 - 30) / 16 for a and ((e + 3 seed) * 40503 % 61 - 30) / 16 for b, c from zero,
  each output within twice its contract bound of the host multiply. The values are multiples of 1/16 whose sums
  are exact in f32, so the device also equals the host loop bit for bit.
- The matmul application's device layer (examples/apps/matmul/src/device_main.cairn, test_app_matmul.py:56-62):
  f16 256 x 512 x 1024 from draw() with seeds 1 and 2, 0 outputs outside the contract.
- C2 (bf16 4096^3) through cf_mma_bf16_device, held to the contract and to BASELINE's 1e-2.
- An enqueued call returns before its stream has run it and may be captured in a HIP graph; a bound stream takes
  the thread's work after what the caller queued there; k = 0 leaves c as it is.
"""

from __future__ import annotations

import ctypes as C
import sys
import time

import numpy as np
import pytest

import helpers as H
from cairn_amd import hip
from cairn_amd import lib as L

pytestmark = pytest.mark.gpu

FORMATS = ["f16", "bf16", "f8e4m3", "f8e5m2"]
DEVICE_SHAPES = [(1, 1, 1, 1), (65, 63, 33, 2), (130, 70, 100, 3), (64, 64, 32, 4), (72, 80, 96, 5), (129, 136, 8, 6),
                 (3, 4, 0, 7)]  # fmt: skip


def say(*what):
    print("[gpu]", *what, flush=True)
    sys.stdout.flush()


def entry(prefix: str, name: str):
    return getattr(L.load(), f"{prefix}_mma_{name}_device")


def views(*arrays):
    """Device copies of host arrays (a zero-length array still gets a valid pointer)."""
    return [hip.Buffer.of(np.ascontiguousarray(x)) for x in arrays]


def checked(name: str, m: int, n: int, k: int, c0: np.ndarray, a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """cf_mma_<name>_device on device views of c0, a, b; returns c."""
    dc, da, db = views(c0, a, b)
    entry("cf", name)(m, n, k, c0.size, dc.ptr, a.size, da.ptr, b.size, db.ptr)
    got = dc.download(c0.shape, np.float32)  # cf_ returned once its stream ran the work
    for x in (dc, da, db):
        x.close()
    return got


@pytest.mark.parametrize("name", FORMATS)
def test_the_checked_device_entry_keeps_the_reference_device_check(name):
    fmt = H.FORMATS[name]
    for m, n, k, seed in DEVICE_SHAPES:
        say(f"cf_mma_{name}_device {m}x{n}x{k} seed {seed}")
        a = H.encode(fmt, H.device_values(m * k, seed, 2654435761)).reshape(m, k)
        b = H.encode(fmt, H.device_values(k * n, seed * 3, 40503)).reshape(k, n)
        c0 = np.zeros((m, n), dtype=np.float32)
        got = checked(name, m, n, k, c0, a, b)
        want = c0.copy()
        assert H.mma(fmt, m, n, k, want, a, b) == 0
        exact, mag = H.gemm_f64(fmt, m, n, k, a, b)
        assert H.outside(got, exact, 2 * H.bound(k, c0, mag)) == 0, (name, m, n, k)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (name, m, n, k)


def test_the_matmul_applications_device_layer_keeps_the_contract():
    """device_main.cairn: x = fill(seed 1), w = fill(seed 2) in f16, out from zero, outside() with slack
    (inner + 1) / 2^22 over sum |x w| (layer.cairn:42-53)."""
    rows, cols, inner = 256, 512, 1024
    x = H.draw(1, rows * inner).astype(np.float16).view(np.uint16).reshape(rows, inner)
    w = H.draw(2, inner * cols).astype(np.float16).view(np.uint16).reshape(inner, cols)
    out = checked("f16", rows, cols, inner, np.zeros((rows, cols), dtype=np.float32), x, w)
    exact, mag = H.exact_product(H.values(H.F16, x), H.values(H.F16, w))
    room = (inner + 1) / 2.0**22 * mag
    broken = int(np.count_nonzero(~(np.abs(out.astype(np.float64) - exact) <= room)))
    say(f"device layer: {rows} x {cols} x {inner}, {broken} outputs outside the contract")
    assert broken == 0


def test_c2_through_the_checked_entry():
    """BASELINE configs[1] (4096^3, A and B ~ N(0, 1/64) in bf16) as emitted code runs it: c += a b into f32 c from
    zero. Every output of 512 sampled rows within its contract bound, and max |got - exact| / sum |a b| <= 1e-2."""
    n = 4096
    rng = np.random.default_rng(4096)
    a = H.normal_bf16(rng, (n, n), 1 / 64)
    b = H.normal_bf16(rng, (n, n), 1 / 64)
    got = checked("bf16", n, n, n, np.zeros((n, n), dtype=np.float32), a, b)
    rows = np.sort(rng.choice(n, 512, replace=False))
    exact, mag = H.exact_product(H.values(H.BF16, a[rows]), H.values(H.BF16, b))
    assert H.outside(got[rows], exact, H.bound(n, np.zeros(1), mag)) == 0
    assert float(np.max(np.abs(got[rows] - exact) / mag)) <= 1e-2


def test_k_zero_leaves_c_and_empty_extents_queue_nothing():
    c0 = (H.tile_values(12, 3) / 2).astype(np.float32).reshape(3, 4)
    empty = np.zeros(0, dtype=np.uint16)
    got = checked("bf16", 3, 4, 0, c0, empty, empty)
    assert np.array_equal(got.view(np.uint32), c0.view(np.uint32))


def queued_ahead(stream: hip.Stream, bufs: list, launches: int = 24) -> None:
    """Several milliseconds of 4096^3 multiplies queued on `stream`, into a buffer of their own."""
    n = 4096
    a, b, c = hip.Buffer(n * n * 2), hip.Buffer(n * n * 2), hip.Buffer(n * n * 2)
    for x in (a, b):
        x.zero()
    bufs += [a, b, c]
    d = L.desc(L.BF16, L.BF16, n, n, n, a.ptr, b.ptr, c.ptr)
    for _ in range(launches):
        L.run(d, stream.handle)


@pytest.mark.parametrize("name", FORMATS)
def test_the_enqueued_entry_queues_on_the_callers_stream_and_never_waits(name):
    fmt = H.FORMATS[name]
    m, n, k = 300, 264, 520
    a = H.encode(fmt, H.tile_values(m * k, 11)).reshape(m, k)
    b = H.encode(fmt, H.tile_values(k * n, 12)).reshape(k, n)
    c0 = (H.tile_values(m * n, 13) / 4).astype(np.float32).reshape(m, n)
    want = c0.copy()
    assert H.mma(fmt, m, n, k, want, a, b) == 0
    stream, bufs = hip.Stream(), []
    queued_ahead(stream, bufs)
    dc, da, db = views(c0, a, b)
    t0 = time.perf_counter()
    entry("cq", name)(stream.handle, m, n, k, c0.size, dc.ptr, a.size, da.ptr, b.size, db.ptr)
    returned = time.perf_counter() - t0
    busy = not stream.idle()
    stream.synchronize()
    got = dc.download(c0.shape, np.float32)
    say(f"cq_mma_{name}_device returned in {returned * 1e6:.0f} us with its stream still busy: {busy}")
    assert busy, "the enqueued entry waited for its stream"
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    for x in (dc, da, db, *bufs):
        x.close()
    stream.close()


def test_the_enqueued_entry_can_be_captured_in_a_graph_and_replayed():
    """cq_ makes no stream or event and allocates nothing, so it records as one kernel node. Each replay adds a b
    once more; with exact data c after r replays is exactly c0 + r a b, checked replay by replay, with eager work
    through the checked entry and host synchronizations between the replays."""
    m, n, k = 256, 512, 256
    a = H.encode(H.BF16, H.tile_values(m * k, 21)).reshape(m, k)
    b = H.encode(H.BF16, H.tile_values(k * n, 22)).reshape(k, n)
    c0 = (H.tile_values(m * n, 23) / 8).astype(np.float32).reshape(m, n)
    exact, _ = H.gemm_f64(H.BF16, m, n, k, a, b)
    stream = hip.Stream()
    dc, da, db = views(c0, a, b)
    cq = entry("cq", "bf16")
    graph = hip.Graph(stream, lambda s: cq(s.handle, m, n, k, c0.size, dc.ptr, a.size, da.ptr, b.size, db.ptr))
    say(f"captured graph: {graph.nodes} node(s)")
    assert graph.nodes == 1
    assert np.array_equal(dc.download(c0.shape, np.float32), c0)  # capture ran nothing
    other = np.zeros((m, n), dtype=np.float32)
    for r in range(1, 4):
        graph.launch(stream)
        stream.synchronize()
        got = dc.download(c0.shape, np.float32)
        assert np.array_equal(got.astype(np.float64), c0.astype(np.float64) + r * exact), r
        eager = checked("bf16", m, n, k, other, a, b)  # eager work on the thread's own stream between replays
        assert np.array_equal(eager.astype(np.float64), exact)
    graph.close()
    for x in (dc, da, db):
        x.close()
    stream.close()


def test_a_bound_stream_takes_the_threads_work_after_what_the_caller_queued():
    """cairn_gemm_device_stream(s): the checked entry runs on s after the caller's work there (a product written into
    c by cairn_gemm_run, queued behind milliseconds of other work) and returns once s has run it; NULL gives the
    thread its own stream back."""
    lib = L.load()
    m, n, k = 256, 256, 256
    a = H.encode(H.BF16, H.tile_values(m * k, 31)).reshape(m, k)
    b = H.encode(H.BF16, H.tile_values(k * n, 32)).reshape(k, n)
    x = H.encode(H.BF16, H.tile_values(m * k, 33)).reshape(m, k)
    stream, bufs = hip.Stream(), []
    dc, da, db, dx = views(np.zeros((m, n), np.float32), a, b, x)
    queued_ahead(stream, bufs)
    L.run(L.desc(L.BF16, L.F32, m, n, k, dx.ptr, db.ptr, dc.ptr), stream.handle)  # c = x b, on the caller's stream
    lib.cairn_gemm_device_stream(stream.handle)
    try:
        lib.cf_mma_bf16_device(m, n, k, m * n, dc.ptr, a.size, da.ptr, b.size, db.ptr)  # c += a b, after it
        assert stream.idle(), "the checked entry returned before its bound stream ran its work"
    finally:
        lib.cairn_gemm_device_stream(None)
    got = dc.download((m, n), np.float32)
    xb, _ = H.gemm_f64(H.BF16, m, n, k, x, b)
    ab, _ = H.gemm_f64(H.BF16, m, n, k, a, b)
    assert np.array_equal(got.astype(np.float64), xb + ab)
    # Unbound: the thread's own stream again, which does not wait for the caller's.
    queued_ahead(stream, bufs)
    again = checked("bf16", m, n, k, np.zeros((m, n), np.float32), a, b)
    assert np.array_equal(again.astype(np.float64), ab)
    stream.synchronize()
    for buf in (dc, da, db, dx, *bufs):
        buf.close()
    stream.close()
