"""Test infrastructure: the CPU oracle (oracle/liboracle.so) through ctypes, the reference's input generators, and the
multiply's contract as a check. Only tests, __graft_entry__.smoke() and bench.py's cpu_baseline leg use the oracle.
"""

from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
ORACLE = ROOT / "oracle" / "liboracle.so"
REF = ROOT / "oracle" / "_ref" / "libcairnref.so"

F32, F16, BF16, F8E4M3, F8E5M2, I8, I32 = range(7)
FORMATS = {"f16": F16, "bf16": BF16, "f8e4m3": F8E4M3, "f8e5m2": F8E5M2}
STORAGE = {F16: np.uint16, BF16: np.uint16, F8E4M3: np.uint8, F8E5M2: np.uint8, F32: np.float32}

_oracle: C.CDLL | None = None


def build_oracle() -> None:
    subprocess.run(["make", "-s", "-C", str(ROOT / "oracle")], check=True, capture_output=True)


def oracle() -> C.CDLL:
    global _oracle
    if _oracle is None:
        if not ORACLE.exists():
            build_oracle()
        o = C.CDLL(str(ORACLE))
        P = C.c_void_p
        sz = C.c_size_t
        o.oracle_decode.restype, o.oracle_decode.argtypes = C.c_double, [C.c_int, C.c_uint32]
        o.oracle_narrow.restype, o.oracle_narrow.argtypes = C.c_uint32, [C.c_int, C.c_double, C.POINTER(C.c_int)]
        o.oracle_quantize_float.restype = C.c_uint32
        o.oracle_quantize_float.argtypes = [C.c_int, C.c_float, C.c_float, C.POINTER(C.c_int)]
        o.oracle_quantize_int.restype = C.c_int64
        o.oracle_quantize_int.argtypes = [C.c_float, C.c_float, C.c_int64, C.c_int64, C.POINTER(C.c_int)]
        o.oracle_shape.restype, o.oracle_shape.argtypes = C.c_int, [sz] * 6
        o.oracle_mma.restype, o.oracle_mma.argtypes = C.c_int, [C.c_int, sz, sz, sz, P, sz, P, sz, P, sz]
        o.oracle_gemm_f64.restype = None
        o.oracle_gemm_f64.argtypes = [C.c_int, C.c_int, C.c_int, sz, sz, sz, P, sz, P, sz, P, P]
        o.oracle_gemm_i8.restype = None
        o.oracle_gemm_i8.argtypes = [C.c_int, C.c_int, sz, sz, sz, P, sz, P, sz, P]
        o.oracle_dequant.restype, o.oracle_dequant.argtypes = None, [sz, sz, P, P, P, P]
        o.oracle_gelu.restype, o.oracle_gelu.argtypes = C.c_double, [C.c_double]
        o.oracle_narrow_f32_array.restype, o.oracle_narrow_f32_array.argtypes = None, [C.c_int, sz, P, P]
        o.oracle_mma_rows.restype = None
        o.oracle_mma_rows.argtypes = [C.c_int, sz, sz, sz, sz, P, P, P, P]
        o.oracle_table.restype, o.oracle_table.argtypes = P, [C.c_int]
        o.oracle_quantize_rows.restype = None
        o.oracle_quantize_rows.argtypes = [C.c_int, C.c_int, C.c_int, sz, sz, P, sz, P, sz, P, C.POINTER(C.c_int)]
        o.oracle_free.restype, o.oracle_free.argtypes = None, [P]
        _oracle = o
    return _oracle


def ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


# ---------------------------------------------------------------- the oracle, numpy in and out


def decode(fmt: int, bits) -> np.ndarray:
    o = oracle()
    return np.array([o.oracle_decode(fmt, int(b)) for b in np.asarray(bits).ravel()]).reshape(np.shape(bits))


def narrow(fmt: int, x: float) -> tuple[int, bool]:
    t = C.c_int()
    b = oracle().oracle_narrow(fmt, float(x), C.byref(t))
    return b, bool(t.value)


def mma(fmt: int, m: int, n: int, k: int, c: np.ndarray, a: np.ndarray, b: np.ndarray) -> int:
    """The reference loop, in place on c (f32). Returns nonzero where the reference traps."""
    return oracle().oracle_mma(fmt, m, n, k, ptr(c), c.size, ptr(a), a.size, ptr(b), b.size)


def gemm_f64(fmt: int, m: int, n: int, k: int, a: np.ndarray, b: np.ndarray, *, trans_a=False, trans_b=False,
             lda=0, ldb=0) -> tuple[np.ndarray, np.ndarray]:  # fmt: skip
    """The exact product in fp64 and sum |a*b|, for small problems (a C loop)."""
    out, mag = np.zeros((m, n)), np.zeros((m, n))
    lda = lda or (m if trans_a else k)
    ldb = ldb or (k if trans_b else n)
    oracle().oracle_gemm_f64(fmt, int(trans_a), int(trans_b), m, n, k, ptr(a), lda, ptr(b), ldb, ptr(out), ptr(mag))
    return out, mag


def gemm_i8(m: int, n: int, k: int, a: np.ndarray, b: np.ndarray, *, trans_a=False, trans_b=False) -> np.ndarray:
    out = np.zeros((m, n), dtype=np.int32)
    lda = m if trans_a else k
    ldb = k if trans_b else n
    oracle().oracle_gemm_i8(int(trans_a), int(trans_b), m, n, k, ptr(a), lda, ptr(b), ldb, ptr(out))
    return out


def dequant(acc: np.ndarray, sa: np.ndarray | None, sb: np.ndarray | None) -> np.ndarray:
    m, n = acc.shape
    out = np.zeros((m, n), dtype=np.uint16)
    acc = np.ascontiguousarray(acc, dtype=np.int32)
    oracle().oracle_dequant(m, n, ptr(acc), ptr(sa), ptr(sb), ptr(out))
    return out


def narrow_array(fmt: int, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(x.shape, dtype=np.uint16)
    oracle().oracle_narrow_f32_array(fmt, x.size, ptr(x), ptr(out))
    return out


def quantize_rows(x_type: int, q_type: int, mode: int, x: np.ndarray, k: int, scale: np.ndarray | None = None
                  ) -> tuple[np.ndarray, np.ndarray, int]:  # fmt: skip
    """The device quantize's contract on the CPU: x is m rows of ldx = x.shape[1] elements (f32, or 16-bit patterns),
    of which the first k are quantized. Returns (q m x k uint8 patterns, the scales, the status bits)."""
    x = np.ascontiguousarray(x)
    m, ldx = x.shape
    q = np.zeros((m, max(k, 1)), dtype=np.uint8)
    s = np.zeros(m, dtype=np.float32) if mode == 0 else np.ascontiguousarray(scale, dtype=np.float32).copy()
    status = C.c_int(0)
    oracle().oracle_quantize_rows(x_type, q_type, mode, m, k, ptr(x), ldx, ptr(q), q.shape[1], ptr(s),
                                  C.byref(status))  # fmt: skip
    return q[:, :k], s, status.value


# ---------------------------------------------------------------- numpy forms used at sizes the C loops cannot reach


def bf16_from_f32(x: np.ndarray) -> np.ndarray:
    """f32 -> bf16 patterns, nearest even, NaN to the quiet 0x7fc0 with its sign (checked against the oracle)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    r = ((u + np.uint32(0x7FFF) + ((u >> 16) & np.uint32(1))) >> 16).astype(np.uint16)
    nan = (u & np.uint32(0x7FFFFFFF)) > np.uint32(0x7F800000)
    r[nan] = (((u[nan] >> 16) & np.uint32(0x8000)) | np.uint32(0x7FC0)).astype(np.uint16)
    return r


def f32_from_bf16(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_from_f16(h: np.ndarray) -> np.ndarray:
    return np.asarray(h, dtype=np.uint16).view(np.float16).astype(np.float32)


def values(fmt: int, bits: np.ndarray) -> np.ndarray:
    """Storage-float patterns as float64 values (exact)."""
    if fmt == BF16:
        return f32_from_bf16(bits).astype(np.float64)
    if fmt == F16:
        return f32_from_f16(bits).astype(np.float64)
    if fmt == F32:
        return np.asarray(bits, dtype=np.float32).astype(np.float64)
    table = decode(fmt, np.arange(256, dtype=np.uint32))
    return table[np.asarray(bits, dtype=np.uint8)]


def normal_bf16(rng: np.random.Generator, shape, std: float) -> np.ndarray:
    return bf16_from_f32(rng.normal(0.0, std, size=shape).astype(np.float32))


def exact_product(av: np.ndarray, bv: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """fp64 a @ b and |a| @ |b| (the magnitude the contract scales with) from operand values, via BLAS."""
    return av @ bv, np.abs(av) @ np.abs(bv)


# ---------------------------------------------------------------- the reference's generators


def mix(x):
    """tests/runtime/tensor_runtime.cpp:69-74 (splitmix-style finalizer), on uint64 arrays."""
    x = np.asarray(x, dtype=np.uint64)
    with np.errstate(over="ignore"):
        x = x ^ (x >> np.uint64(31))
        x = x * np.uint64(0x7FB5D329728EA185)
        x = x ^ (x >> np.uint64(27))
    return x


def tile_values(count: int, seed: int) -> np.ndarray:
    """(mix(seed + e) % 61 - 30) / 16: multiples of 1/16 in [-1.875, 1.875] (tensor_runtime.cpp:76-87)."""
    h = mix(np.arange(count, dtype=np.uint64) + np.uint64(seed))
    return ((h % np.uint64(61)).astype(np.int64) - 30).astype(np.float64) / 16.0


def device_values(count: int, seed: int, mul: int) -> np.ndarray:
    """The device test's draw (tests/soundness/test_tensor.py:201-202): ((e + seed) * mul % 61 - 30) / 16."""
    e = np.arange(count, dtype=np.uint64) + np.uint64(seed)
    with np.errstate(over="ignore"):
        h = e * np.uint64(mul)
    return ((h % np.uint64(61)).astype(np.int64) - 30).astype(np.float64) / 16.0


def draw(seed: int, count: int) -> np.ndarray:
    """examples/apps/matmul/src/layer.cairn:8-11: h = (e + seed) * 0x9e37.. ^ ((e * 0xbf58..) >> 31);
    (h % 2048 - 1024) / 1024 in f32."""
    e = np.arange(count, dtype=np.uint64)
    with np.errstate(over="ignore"):
        h = ((e + np.uint64(seed)) * np.uint64(0x9E3779B97F4A7C15)) ^ ((e * np.uint64(0xBF58476D1CE4E5B9)) >> np.uint64(31))
    return (((h % np.uint64(2048)).astype(np.int64) - 1024).astype(np.float32) / np.float32(1024.0))


def encode(fmt: int, v: np.ndarray) -> np.ndarray:
    """Values exactly representable in fmt (the generators' multiples of 1/16 or 1/1024) as patterns."""
    v = np.asarray(v, dtype=np.float64)
    if fmt == BF16:
        return bf16_from_f32(v.astype(np.float32))
    if fmt == F16:
        return v.astype(np.float16).view(np.uint16)
    if fmt == F32:
        return v.astype(np.float32)
    out = np.empty(v.shape, dtype=np.uint8)
    flat = out.ravel()
    for i, x in enumerate(v.ravel()):
        bits, trapped = narrow(fmt, float(x))
        assert not trapped
        flat[i] = bits
    return out


# ---------------------------------------------------------------- the contract


def bound(k: int, c_old: np.ndarray, mag: np.ndarray, factor: float = 1.0) -> np.ndarray:
    """(k + 1) * 2^-22 * (|c| + sum |a * b|): src/cairn/compiler/device/tensor.py:10-12,32."""
    return factor * (k + 1) * 2.0**-22 * (np.abs(c_old.astype(np.float64)) + mag)


def outside(got: np.ndarray, want: np.ndarray, room: np.ndarray) -> int:
    """How many outputs lie outside their bound (a NaN counts as outside)."""
    d = np.abs(got.astype(np.float64) - want)
    return int(np.count_nonzero(~(d <= room)))
