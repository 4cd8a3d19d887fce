"""The MFMA fragments (include/cairn/cairn_fragment.hpp) on the device, against the host model and the reference loop.

tests/cpp/fragment_device.hip holds kernels written with the fragments as CAIRN-emitted cooperative code uses them;
__graft_entry__.build() compiles it into tests/cpp/libfragment_device.so. The data make every sum exact in f32
(multiples of 1/16 in [-2, 2]; int8 sums are exact anyway), so whatever order the matrix cores add in, the device
must equal the host model, which adds in increasing k as the reference loop does (cairn_fragment.hpp's contract):

- one wave through every shape and operand type, over several k-steps, with tiles row-major, padded, swizzled or
  stored by columns, read from global memory or from LDS;
- the lane share: which element each lane's value v is (get), and that set and store write each element once;
- a whole GEMM in the shape of the reference's examples/tensor/tile64.cairn on the reference's device shapes,
  bit for bit equal to the host reference loop.
"""

from __future__ import annotations

import ctypes as C
import sys
from pathlib import Path

import numpy as np
import pytest

import helpers as H
from cairn_amd import hip

pytestmark = pytest.mark.gpu
LIB = Path(__file__).resolve().parent / "cpp" / "libfragment_device.so"
P, I = C.c_void_p, C.c_int


def say(*what):
    print("[gpu]", *what, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def lib():
    if not LIB.exists():
        pytest.fail(f"{LIB} is not built: run __graft_entry__.build()")
    lib = C.CDLL(str(LIB))
    for name in ("frag_wave_bf16_32x32x16", "frag_wave_f16_32x32x16", "frag_wave_bf16_16x16x32",
                 "frag_wave_f16_16x16x32", "frag_wave_i8_32x32x32"):  # fmt: skip
        getattr(lib, name).argtypes = [P, P, P, P, P, P, P, I, I, I, I]
    for name in ("frag_share_bf16_32x32x16", "frag_share_bf16_16x16x32"):
        getattr(lib, name).argtypes = [P, P, P, P]
    lib.frag_tile_gemm.argtypes = [I, I, I, I, P, P, P]
    return lib


def offsets(rows: int, cols: int, pitch: int, by_columns: int, swizzle: int) -> np.ndarray:
    """The tile layout of fragment_device.hip's Tile: offset of each (r, c)."""
    r, c = np.meshgrid(np.arange(rows), np.arange(cols), indexing="ij")
    o = c * pitch + r if by_columns else r * pitch + c
    if swizzle:
        o = o ^ ((o >> 3) & (((1 << swizzle) - 1) << 3))
    return o


def values(kind: str, count: int, seed: int) -> tuple[np.ndarray, np.ndarray]:
    """(storage array, f64 values) of count exact operands."""
    rng = np.random.default_rng(seed)
    if kind == "i8":
        v = rng.integers(-127, 128, count).astype(np.int8)
        return v, v.astype(np.float64)
    x = rng.integers(-32, 33, count) / 16.0
    fmt = H.BF16 if kind == "bf16" else H.F16
    return H.encode(fmt, x), x


SHAPES = {"bf16_32x32x16": ("bf16", 32, 32, 16), "f16_32x32x16": ("f16", 32, 32, 16),
          "bf16_16x16x32": ("bf16", 16, 16, 32), "f16_16x16x32": ("f16", 16, 16, 32),
          "i8_32x32x32": ("i8", 32, 32, 32)}  # fmt: skip
# (A tile, B tile, C tile) as (pitch extra, by columns, swizzle); pitches are the tile's own width plus the extra.
LAYOUTS = [((0, 0, 0), (0, 0, 0), (0, 0, 0)), ((8, 0, 0), (8, 1, 0), (4, 0, 0)), ((0, 0, 1), (0, 0, 2), (0, 1, 0)),
           ((16, 0, 0), (0, 1, 0), (0, 0, 0))]  # fmt: skip


@pytest.mark.parametrize("via_lds", [0, 1])
@pytest.mark.parametrize("shape", list(SHAPES))
def test_one_wave_equals_the_host_model_through_every_layout(lib, shape, via_lds):
    kind, m, n, k = SHAPES[shape]
    steps = 3
    f = getattr(lib, f"frag_wave_{shape}")
    for li, (la, lb, lc) in enumerate(LAYOUTS):
        if kind == "i8" and (la[2] or lb[2]):
            continue  # a swizzle of 8-byte units would split int8 runs differently; the 16-bit cases cover it
        ta = (steps * k + la[0] if not la[1] else m + la[0], la[1], la[2])
        tb = (n + lb[0] if not lb[1] else steps * k + lb[0], lb[1], lb[2])
        tc = (n + lc[0] if not lc[1] else m + lc[0], lc[1], lc[2])
        oa, ob, oc = offsets(m, steps * k, *ta), offsets(steps * k, n, *tb), offsets(m, n, *tc)
        av, ax = values(kind, m * steps * k, 10 + li)
        bv, bx = values(kind, steps * k * n, 20 + li)
        a = np.zeros(oa.max() + 1, dtype=av.dtype)
        b = np.zeros(ob.max() + 1, dtype=bv.dtype)
        a[oa.ravel()] = av
        b[ob.ravel()] = bv
        c0 = (np.random.default_rng(30 + li).integers(-16, 17, (m, n)) / (1 if kind == "i8" else 4.0))
        cdt = np.int32 if kind == "i8" else np.float32
        c = np.zeros(oc.max() + 1, dtype=cdt)
        c[oc.ravel()] = c0.ravel().astype(cdt)
        want = c0 + ax.reshape(m, steps * k) @ bx.reshape(steps * k, n)
        dc, da, db = hip.Buffer.of(c), hip.Buffer.of(a), hip.Buffer.of(b)
        say(f"frag wave {shape} layout {li} lds {via_lds}")
        ints = [np.array(x, dtype=np.int32) for x in (ta, tb, tc)]
        status = f(None if kind == "i8" else dc.ptr, dc.ptr if kind == "i8" else None, da.ptr, db.ptr,
                   *[x.ctypes.data_as(P) for x in ints], steps, a.size, b.size, via_lds)  # fmt: skip
        assert status == 0
        hip.synchronize()
        got = dc.download((c.size,), cdt)[oc].astype(np.float64)
        for x in (dc, da, db):
            x.close()
        assert np.array_equal(got, want), (shape, li, via_lds)


def lane_share(m: int, lane: int, v: int) -> tuple[int, int]:
    """The element value v of lane l is, as cairn_fragment.hpp states the device's share."""
    if m == 32:
        return 8 * (v // 4) + 4 * (lane // 32) + v % 4, lane % 32
    return 4 * (lane // 16) + v, lane % 16


@pytest.mark.parametrize("shape", ["bf16_32x32x16", "bf16_16x16x32"])
def test_each_lane_holds_the_elements_the_header_states(lib, shape):
    kind, m, n, k = SHAPES[shape]
    nv = m * n // 64
    av, ax = values(kind, m * k, 41)
    bv, bx = values(kind, k * n, 42)
    want = ax.reshape(m, k) @ bx.reshape(k, n)
    dg, dc, da, db = hip.Buffer(64 * nv * 4), hip.Buffer(m * n * 4), hip.Buffer.of(av), hip.Buffer.of(bv)
    dc.zero()
    say(f"frag share {shape}")
    assert getattr(lib, f"frag_share_{shape}")(dg.ptr, dc.ptr, da.ptr, db.ptr) == 0
    hip.synchronize()
    got = dg.download((64, nv), np.float32)
    stored = dc.download((m, n), np.float32)
    for x in (dg, dc, da, db):
        x.close()
    seen = np.zeros((m, n), dtype=int)
    for lane in range(64):
        for v in range(nv):
            r, c = lane_share(m, lane, v)
            assert got[lane, v] == want[r, c], (shape, lane, v)
            assert stored[r, c] == 1000 * lane + v, (shape, lane, v)
            seen[r, c] += 1
    assert np.all(seen == 1)


DEVICE_SHAPES = [(1, 1, 1, 1), (65, 63, 33, 2), (130, 70, 100, 3), (64, 64, 32, 4), (72, 80, 96, 5), (129, 136, 8, 6),
                 (3, 4, 0, 7)]  # fmt: skip


@pytest.mark.parametrize("name", ["bf16", "f16"])
def test_a_tile64_shaped_fragment_gemm_equals_the_host_loop(lib, name):
    fmt = H.FORMATS[name]
    for m, n, k, seed in DEVICE_SHAPES:
        a = H.encode(fmt, H.device_values(m * k, seed, 2654435761)).reshape(m, k)
        b = H.encode(fmt, H.device_values(k * n, seed * 3, 40503)).reshape(k, n)
        c0 = (H.tile_values(m * n, 99 + seed) / 2).astype(np.float32).reshape(m, n)
        want = c0.copy()
        assert H.mma(fmt, m, n, k, want, a, b) == 0
        dc, da, db = hip.Buffer.of(c0), hip.Buffer.of(a if a.size else np.zeros(1, np.uint16)), \
            hip.Buffer.of(b if b.size else np.zeros(1, np.uint16))  # fmt: skip
        say(f"frag tile gemm {name} {m}x{n}x{k}")
        assert lib.frag_tile_gemm(fmt, m, n, k, dc.ptr, da.ptr, db.ptr) == 0
        hip.synchronize()
        got = dc.download((m, n), np.float32)
        for x in (dc, da, db):
            x.close()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (name, m, n, k)
