"""Write tests/golden/reference.npz: input/output vectors of the reference's own host multiply and storage floats,
computed by the reference's header compiled into oracle/_ref/libcairnref.so (oracle/ref_shim.cpp, oracle/Makefile).

Run in a container where /root/reference is mounted (make -C oracle builds oracle/_ref first):

    python tests/golden/make_golden.py

The fixture is data only (inputs and the reference's outputs). The cases follow the reference's own tests:

- mma_*: tests/soundness/test_tensor.py:48-85 (random finite patterns, |v| <= 448, 1e6 for bf16; c ~ U(-4, 4) in f32;
  the SHAPES list), for each storage float and for the f32 instance of the template (config C1's loop);
- tile_*: tests/runtime/tensor_runtime.cpp:69-110 (the mix() generator, (h % 61 - 30) / 16, old c (h % 9 - 4) / 4, on
  the tail shapes);
- app_*: examples/apps/matmul/src/layer.cairn:6-23 and main.cairn:9-40 (draw(seed, e), f16, 200 x 136 x 72 with seeds
  1 and 2, and the 2 x 2 x 3 case with seeds 7 and 8);
- narrow_*, quantize_*, decode_*: cr::fp::narrow / quantize / operator double on ties, exact values, random doubles
  and every 8-bit pattern (tests/language/test_storage_floats.py:91-160 is the model).
"""

from __future__ import annotations

import ctypes as C
import math
import random
import struct
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT / "tests"))
import helpers as H  # noqa: E402

FORMATS = {"f16": (H.F16, C.c_uint16, np.uint16, 16), "bf16": (H.BF16, C.c_uint16, np.uint16, 16),
           "f8e4m3": (H.F8E4M3, C.c_uint8, np.uint8, 8), "f8e5m2": (H.F8E5M2, C.c_uint8, np.uint8, 8)}  # fmt: skip
SHAPES = [(1, 1, 1), (3, 5, 7), (8, 8, 8), (17, 3, 33), (2, 40, 5), (4, 4, 0), (0, 3, 3), (12, 13, 64)]
TILE_SHAPES = [(1, 1, 1), (64, 64, 32), (65, 63, 33), (17, 200, 64), (3, 129, 31), (72, 80, 96)]


def ref() -> C.CDLL:
    if not H.REF.exists():
        raise SystemExit(f"{H.REF} is missing: build it with `make -C oracle` where /root/reference is mounted")
    return C.CDLL(str(H.REF))


def f32(x: float) -> float:
    return struct.unpack("<f", struct.pack("<f", x))[0]


def mma(lib, name: str, m: int, n: int, k: int, c: np.ndarray, a: np.ndarray, b: np.ndarray) -> np.ndarray:
    f = getattr(lib, f"ref_mma_{name}")
    P, S = C.c_void_p, C.c_size_t
    f.argtypes = [S, S, S, P, S, P, S, P, S]
    out = np.ascontiguousarray(c, dtype=np.float32).copy()
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    f(m, n, k, out.ctypes.data_as(P), out.size, a.ctypes.data_as(P), a.size, b.ctypes.data_as(P), b.size)
    return out


def finite_patterns(fmt: int, rng: random.Random, count: int, limit: float, width: int) -> list[int]:
    out = []
    while len(out) < count:
        p = rng.randrange(1 << width)
        v = H.oracle().oracle_decode(fmt, p)
        if v == v and abs(v) <= limit:
            out.append(p)
    return out


def main() -> None:
    lib = ref()
    data: dict[str, np.ndarray] = {}

    # mma_<fmt>_<i>: the reference test's random patterns on SHAPES.
    for name, (fmt, _, dtype, width) in FORMATS.items():
        rng = random.Random(f"mma-{name}")
        limit = 448.0 if name != "bf16" else 1e6
        for i, (m, n, k) in enumerate(SHAPES):
            a = np.array(finite_patterns(fmt, rng, m * k, limit, width), dtype=dtype)
            b = np.array(finite_patterns(fmt, rng, k * n, limit, width), dtype=dtype)
            c = np.array([f32(rng.uniform(-4, 4)) for _ in range(m * n)], dtype=np.float32)
            key = f"mma_{name}_{i}"
            data[key + "_shape"] = np.array([m, n, k], dtype=np.int64)
            data[key + "_a"], data[key + "_b"], data[key + "_c"] = a, b, c
            data[key + "_out"] = mma(lib, name, m, n, k, c, a, b)
    # f32: config C1's loop at a small size (uniform [-1, 1) inputs, c zero).
    rng = np.random.default_rng(512)
    for i, (m, n, k) in enumerate([(5, 7, 9), (32, 48, 40)]):
        a = rng.uniform(-1, 1, m * k).astype(np.float32)
        b = rng.uniform(-1, 1, k * n).astype(np.float32)
        c = np.zeros(m * n, dtype=np.float32)
        key = f"mma_f32_{i}"
        data[key + "_shape"] = np.array([m, n, k], dtype=np.int64)
        data[key + "_a"], data[key + "_b"], data[key + "_c"] = a, b, c
        data[key + "_out"] = mma(lib, "f32", m, n, k, c, a, b)

    # tile_<fmt>_<i>: tensor_runtime.cpp's generator on its tail shapes.
    for name, (fmt, _, dtype, _) in FORMATS.items():
        for i, (m, n, k) in enumerate(TILE_SHAPES):
            a = H.encode(fmt, H.tile_values(m * k, 1 + m))
            b = H.encode(fmt, H.tile_values(k * n, 7 + n))
            h = H.mix(np.arange(m * n, dtype=np.uint64) + np.uint64(99))
            c = (((h % np.uint64(9)).astype(np.int64) - 4).astype(np.float32) / np.float32(4.0))
            key = f"tile_{name}_{i}"
            data[key + "_shape"] = np.array([m, n, k], dtype=np.int64)
            data[key + "_a"], data[key + "_b"], data[key + "_c"] = a, b, c
            data[key + "_out"] = mma(lib, name, m, n, k, c, a, b)

    # app_*: the matmul example's f16 layer and its written-order test.
    for key, (m, n, k, sa, sb) in {"app_layer": (200, 136, 72, 1, 2), "app_order": (2, 2, 3, 7, 8)}.items():
        a = H.draw(sa, m * k).astype(np.float16).view(np.uint16)
        b = H.draw(sb, k * n).astype(np.float16).view(np.uint16)
        c = np.zeros(m * n, dtype=np.float32)
        data[key + "_shape"] = np.array([m, n, k], dtype=np.int64)
        data[key + "_a"], data[key + "_b"], data[key + "_c"] = a, b, c
        data[key + "_out"] = mma(lib, "f16", m, n, k, c, a, b)

    # Storage floats.
    for name, (fmt, ctype, dtype, width) in FORMATS.items():
        dec = getattr(lib, f"ref_decode_{name}")
        dec.restype, dec.argtypes = C.c_double, [ctype]
        nar = getattr(lib, f"ref_narrow_{name}")
        nar.restype, nar.argtypes = ctype, [C.c_double]
        qua = getattr(lib, f"ref_quantize_{name}")
        qua.restype, qua.argtypes = ctype, [C.c_float, C.c_float]
        pats = np.arange(256) if width == 8 else np.array(sorted(set(random.Random(name).sample(range(65536), 800))
                                                                  | {0, 1, 0x7BFF, 0x7C00, 0x7C01, 0x7F7F, 0x7F80, 0x8000, 0xFFFF}))  # fmt: skip
        data[f"decode_{name}_bits"] = pats.astype(np.uint32)
        data[f"decode_{name}_value"] = np.array([dec(int(p)) for p in pats], dtype=np.float64)
        rng = random.Random(20260922 + width)
        xs = [0.0, -0.0, 5e-324, 1e308, -1e308, math.inf, -math.inf, math.nan, 1.0 / 3.0]
        for p in range(0, 1 << width, 1 if width == 8 else 211):
            v = H.oracle().oracle_decode(fmt, p)
            if v == v and not math.isinf(v):
                xs += [v, math.nextafter(v, math.inf), math.nextafter(v, -math.inf)]
        for _ in range(800):
            xs.append(rng.choice((-1, 1)) * math.ldexp(rng.random(), rng.randint(-150, 20)))
        if name == "f8e4m3":  # past 464 the reference traps (no infinity): those are not vectors
            xs = [x for x in xs if not (math.isinf(x) or abs(x) > 464.0)]
        data[f"narrow_{name}_x"] = np.array(xs, dtype=np.float64)
        data[f"narrow_{name}_bits"] = np.array([nar(x) for x in xs], dtype=np.uint32)
        qx, qs = [], []
        for _ in range(800):
            qx.append(f32(rng.uniform(-2, 2) * 500.0))
            qs.append(rng.choice([1.0, 0.25, 3.0, 1e-3, 7.3e-5, 0.37]))
        qx += [math.inf, -math.inf, math.nan, -0.0, 2.5, -2.5]
        qs += [1.0, 1.0, 1.0, 1.0, 1.0, 1.0]
        data[f"quantize_{name}_x"] = np.array(qx, dtype=np.float32)
        data[f"quantize_{name}_scale"] = np.array(qs, dtype=np.float32)
        data[f"quantize_{name}_bits"] = np.array([qua(x, s) for x, s in zip(qx, qs)], dtype=np.uint32)
    qi = lib.ref_quantize_i8
    qi.restype, qi.argtypes = C.c_int8, [C.c_float, C.c_float]
    rng = random.Random(11)
    qx = [f32(rng.uniform(-300, 300)) for _ in range(800)] + [-2.5, 500.0, -0.5, 0.5, 1.5, 126.5, -128.5, math.inf]
    qs = [rng.choice([1.0, 0.5, 2.0, 0.37]) for _ in range(800)] + [1.0, 2.0, 1.0, 1.0, 1.0, 1.0, 1.0, 1.0]
    data["quantize_i8_x"] = np.array(qx, dtype=np.float32)
    data["quantize_i8_scale"] = np.array(qs, dtype=np.float32)
    data["quantize_i8_value"] = np.array([qi(x, s) for x, s in zip(qx, qs)], dtype=np.int8)

    out = HERE / "reference.npz"
    np.savez_compressed(out, **data)
    print(f"wrote {out} ({out.stat().st_size} bytes, {len(data)} arrays)")


if __name__ == "__main__":
    main()
