"""The CPU oracle (oracle/oracle.c) pinned before anything is checked against it.

- Golden vectors written by the reference's own header compiled into oracle/_ref (tests/golden/make_golden.py):
  the host multiply on the reference test's shapes and generators, and the storage-float conversions; bit for bit.
- Where oracle/_ref is built here, fresh random cases against it too.
- An exact model: the written order replayed in Python with every f32 rounding done by struct, and the contract bound
  against the exact rational sum (as tests/soundness/test_tensor.py:76-85 states it).
- Known answers the reference's docs state (docs/numerics.md:31-32), numpy's float16 for f16, exhaustive 8-bit
  decode against the format definitions, the int8 product against numpy's exact integers.
- Planted mistakes (a reversed summation order, a dropped rounding, a transposed operand) fail these checks.
"""

from __future__ import annotations

import ctypes as C
import math
import random
import struct
from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest

import helpers as H

GOLDEN = Path(__file__).resolve().parent / "golden" / "reference.npz"
NAMES = {"f16": H.F16, "bf16": H.BF16, "f8e4m3": H.F8E4M3, "f8e5m2": H.F8E5M2, "f32": H.F32}


@pytest.fixture(scope="module")
def golden():
    with np.load(GOLDEN, allow_pickle=False) as d:
        return {k: d[k] for k in d.files}


def cases(golden, prefix):
    keys = sorted({k.rsplit("_", 1)[0] for k in golden if k.startswith(prefix) and k.endswith("_shape")})
    return [(k, *golden[k + "_shape"].tolist()) for k in keys]


def f32(x: float) -> float:
    return struct.unpack("<f", struct.pack("<f", x))[0]


def bits32(a: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32).view(np.uint32)


# ------------------------------------------------------------------ the host multiply


@pytest.mark.parametrize("prefix", ["mma_", "tile_", "app_"])
def test_the_oracle_multiply_equals_the_reference_bit_for_bit(golden, prefix):
    found = cases(golden, prefix)
    assert found
    for key, m, n, k in found:
        fmt = NAMES[key.split("_")[1]] if prefix != "app_" else H.F16
        c = golden[key + "_c"].copy()
        assert H.mma(fmt, m, n, k, c, golden[key + "_a"], golden[key + "_b"]) == 0
        assert np.array_equal(bits32(c), bits32(golden[key + "_out"])), key


def replay(fmt, m, n, k, c, a, b):
    """The written order with Python floats: acc = f32(acc + f32(x * y)), p upward (test_tensor.py:79-80)."""
    av, bv = H.values(fmt, a), H.values(fmt, b)
    out = c.astype(np.float64).copy()
    for i in range(m):
        for j in range(n):
            acc = float(out[i * n + j])
            for p in range(k):
                acc = f32(acc + f32(float(av[i * k + p]) * float(bv[p * n + j])))
            out[i * n + j] = acc
    return out.astype(np.float32)


def test_the_golden_order_is_the_written_order_and_a_planted_reversal_fails(golden):
    """The exact Python replay of the written order equals the golden output; the same replay with p running
    downward (a plausible mistake) does not, so the vectors pin the order."""
    key = "mma_bf16_7"  # 12 x 13 x 64
    m, n, k = golden[key + "_shape"].tolist()
    a, b, c = golden[key + "_a"], golden[key + "_b"], golden[key + "_c"]
    want = golden[key + "_out"]
    assert np.array_equal(bits32(replay(H.BF16, m, n, k, c, a, b)), bits32(want))
    av, bv = H.values(H.BF16, a), H.values(H.BF16, b)
    reversed_ = c.astype(np.float64).copy()
    for i in range(m):
        for j in range(n):
            acc = float(reversed_[i * n + j])
            for p in reversed(range(k)):
                acc = f32(acc + f32(float(av[i * k + p]) * float(bv[p * n + j])))
            reversed_[i * n + j] = acc
    assert not np.array_equal(bits32(reversed_.astype(np.float32)), bits32(want))


def test_a_planted_transposed_operand_and_a_dropped_rounding_fail(golden):
    key = "mma_f16_7"
    m, n, k = golden[key + "_shape"].tolist()
    a, b, c = golden[key + "_a"], golden[key + "_b"], golden[key + "_c"]
    want = golden[key + "_out"]
    # products and sums in double, rounded once at the end: no longer the reference's bits
    exact = (c.astype(np.float64).reshape(m, n) + H.values(H.F16, a).reshape(m, k) @ H.values(H.F16, b).reshape(k, n))
    assert not np.array_equal(bits32(exact.astype(np.float32).ravel()), bits32(want))
    # a square case read with b transposed
    key = "mma_f16_2"  # 8 x 8 x 8
    m, n, k = golden[key + "_shape"].tolist()
    c = golden[key + "_c"].copy()
    bt = golden[key + "_b"].reshape(k, n).T.copy().ravel()
    H.mma(H.F16, m, n, k, c, golden[key + "_a"], bt)
    assert not np.array_equal(bits32(c), bits32(golden[key + "_out"]))


@pytest.mark.parametrize("name", ["f16", "bf16", "f8e4m3", "f8e5m2"])
def test_the_oracle_is_its_written_order_and_within_the_contract_on_fresh_patterns(name):
    fmt = NAMES[name]
    rng = random.Random(f"oracle-{name}")
    width = 16 if name in ("f16", "bf16") else 8
    limit = 448.0 if name != "bf16" else 1e6
    for m, n, k in [(3, 5, 7), (2, 4, 33)]:
        def pats(count):
            out = []
            while len(out) < count:
                p = rng.randrange(1 << width)
                v = H.oracle().oracle_decode(fmt, p)
                if v == v and abs(v) <= limit:
                    out.append(p)
            return np.array(out, dtype=H.STORAGE[fmt])
        a, b = pats(m * k), pats(k * n)
        c = np.array([f32(rng.uniform(-4, 4)) for _ in range(m * n)], dtype=np.float32)
        got = c.copy()
        H.mma(fmt, m, n, k, got, a, b)
        assert np.array_equal(bits32(got), bits32(replay(fmt, m, n, k, c, a, b)))
        av, bv = H.values(fmt, a), H.values(fmt, b)
        for i in range(m):
            for j in range(n):
                exact, mag = Fraction(float(c[i * n + j])), abs(Fraction(float(c[i * n + j])))
                for p in range(k):
                    prod = Fraction(float(av[i * k + p])) * Fraction(float(bv[p * n + j]))
                    exact += prod
                    mag += abs(prod)
                assert abs(Fraction(float(got[i * n + j])) - exact) <= (k + 1) * Fraction(1, 2**22) * mag


@pytest.mark.skipif(not H.REF.exists(), reason="oracle/_ref is built only where the reference is mounted")
def test_the_oracle_multiply_equals_the_compiled_reference_on_fresh_random_cases():
    ref = C.CDLL(str(H.REF))
    P, S = C.c_void_p, C.c_size_t
    rng = np.random.default_rng(99)
    for name in ("f16", "bf16", "f8e4m3", "f8e5m2", "f32"):
        fmt = NAMES[name]
        f = getattr(ref, f"ref_mma_{name}")
        f.argtypes = [S, S, S, P, S, P, S, P, S]
        for m, n, k in [(17, 23, 41), (1, 64, 100), (40, 3, 1)]:
            if fmt == H.F32:
                a = rng.uniform(-1, 1, m * k).astype(np.float32)
                b = rng.uniform(-1, 1, k * n).astype(np.float32)
            else:
                a = H.encode(fmt, np.round(rng.uniform(-4, 4, m * k) * 16) / 16)
                b = H.encode(fmt, np.round(rng.uniform(-4, 4, k * n) * 16) / 16)
            c = rng.uniform(-2, 2, m * n).astype(np.float32)
            want = c.copy()
            f(m, n, k, want.ctypes.data_as(P), want.size, a.ctypes.data_as(P), a.size, b.ctypes.data_as(P), b.size)
            got = c.copy()
            H.mma(fmt, m, n, k, got, a, b)
            assert np.array_equal(bits32(got), bits32(want)), (name, m, n, k)


def test_the_extents_check_traps_where_the_reference_traps():
    assert H.oracle().oracle_shape(2, 3, 3, 6, 6, 9) == 0
    assert H.oracle().oracle_shape(2, 3, 3, 6, 6, 6) != 0  # b holds 6, not 3 * 3 (test_tensor.py:109-119)
    assert H.oracle().oracle_shape(2**63, 2, 1, 0, 2**63, 2) != 0  # m * n overflows
    c = np.arange(6, dtype=np.float32)
    assert H.mma(H.F16, 2, 3, 0, c, np.zeros(0, np.uint16), np.zeros(0, np.uint16)) == 0
    assert np.array_equal(c, np.arange(6, dtype=np.float32))  # k = 0 leaves c as it is (main.cairn:42-49)


# ------------------------------------------------------------------ storage floats


@pytest.mark.parametrize("name", ["f16", "bf16", "f8e4m3", "f8e5m2"])
def test_decode_equals_the_reference(golden, name):
    fmt = NAMES[name]
    got = H.decode(fmt, golden[f"decode_{name}_bits"])
    want = golden[f"decode_{name}_value"]
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint64), want[~nan].view(np.uint64))


@pytest.mark.parametrize("name", ["f16", "bf16", "f8e4m3", "f8e5m2"])
def test_narrow_equals_the_reference(golden, name):
    fmt = NAMES[name]
    xs, want = golden[f"narrow_{name}_x"], golden[f"narrow_{name}_bits"]
    got = [H.narrow(fmt, float(x))[0] for x in xs]
    assert [int(g) for g in got] == [int(w) for w in want]


@pytest.mark.parametrize("name", ["f16", "bf16", "f8e4m3", "f8e5m2"])
def test_quantize_equals_the_reference(golden, name):
    fmt = NAMES[name]
    o = H.oracle()
    t = C.c_int()
    xs, ss, want = golden[f"quantize_{name}_x"], golden[f"quantize_{name}_scale"], golden[f"quantize_{name}_bits"]
    got = [o.oracle_quantize_float(fmt, float(x), float(s), C.byref(t)) for x, s in zip(xs, ss)]
    assert got == [int(w) for w in want]


def test_quantize_int8_equals_the_reference(golden):
    o = H.oracle()
    t = C.c_int()
    xs, ss, want = golden["quantize_i8_x"], golden["quantize_i8_scale"], golden["quantize_i8_value"]
    got = [o.oracle_quantize_int(float(x), float(s), -128, 127, C.byref(t)) for x, s in zip(xs, ss)]
    assert got == [int(w) for w in want]


def test_the_known_answers_of_the_reference_docs():
    """docs/numerics.md:31-32."""
    assert H.narrow(H.F16, 1.0 / 3.0)[0] == 0x3555
    one, half = H.narrow(H.BF16, 1.0)[0], H.narrow(H.BF16, 0.5)[0]
    mean = f32((f32(H.decode(H.BF16, [one])[0]) + f32(H.decode(H.BF16, [half])[0])) / 2.0)
    assert f32(H.decode(H.BF16, [H.narrow(H.BF16, mean)[0]])[0]) == 0.75
    o, t = H.oracle(), C.c_int()
    assert o.oracle_quantize_int(-2.5, 1.0, -128, 127, C.byref(t)) == -2  # ties to even
    assert o.oracle_quantize_int(500.0, 2.0, -128, 127, C.byref(t)) == 127  # saturates
    o.oracle_quantize_int(1.0, 0.0, -128, 127, C.byref(t))
    assert t.value  # a scale that is not positive traps
    H.narrow(H.F8E4M3, 480.0)
    assert H.narrow(H.F8E4M3, 480.0)[1]  # past 464 E4M3 has no answer: a trap
    assert H.narrow(H.F8E4M3, 464.0) == (0x7E, False)  # the tie rounds to the even 448
    assert H.narrow(H.F16, 70000.0)[0] == 0x7C00  # f16 overflows to infinity


def test_f16_agrees_with_numpy_binary16():
    rng = np.random.default_rng(7)
    xs = np.ldexp(rng.random(4000), rng.integers(-30, 17, 4000)) * rng.choice([-1.0, 1.0], 4000)
    want = xs.astype(np.float16).view(np.uint16)
    got = np.array([H.narrow(H.F16, float(x))[0] for x in xs], dtype=np.uint16)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("name,e,m,infinite", [("f8e4m3", 4, 3, False), ("f8e5m2", 5, 2, True)])
def test_every_8bit_pattern_decodes_to_its_definition(name, e, m, infinite):
    """OCP E4M3 / E5M2 from their definitions, exactly."""
    bias = 2 ** (e - 1) - 1
    for p in range(256):
        sign = -1.0 if p & 0x80 else 1.0
        exp, frac = (p >> m) & ((1 << e) - 1), p & ((1 << m) - 1)
        if exp == (1 << e) - 1 and (infinite or frac == (1 << m) - 1):
            want = math.nan if (frac or not infinite) else sign * math.inf
        elif exp == 0:
            want = sign * math.ldexp(frac, 1 - bias - m)
        else:
            want = sign * math.ldexp((1 << m) + frac, exp - bias - m)
        got = H.decode(NAMES[name], [p])[0]
        assert (math.isnan(got) and math.isnan(want)) or got == want, hex(p)


def test_the_bf16_array_rounding_equals_the_oracle():
    """tests/helpers.bf16_from_f32 (used at sizes the C loop cannot reach) against the oracle's narrow<bf16>."""
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.normal(0, 1, 20000), rng.normal(0, 1e30, 2000), [np.inf, -np.inf, np.nan, -0.0, 3.4e38]])
    x = x.astype(np.float32)
    assert np.array_equal(H.bf16_from_f32(x), H.narrow_array(H.BF16, x))


# ------------------------------------------------------------------ north-star additions


def test_the_int8_product_is_numpy_exact():
    rng = np.random.default_rng(1)
    for ta in (False, True):
        for tb in (False, True):
            m, n, k = 37, 29, 300
            a = rng.integers(-128, 128, (k, m) if ta else (m, k), dtype=np.int8)
            b = rng.integers(-128, 128, (n, k) if tb else (k, n), dtype=np.int8)
            want = (a.T if ta else a).astype(np.int64) @ (b.T if tb else b).astype(np.int64)
            assert np.array_equal(H.gemm_i8(m, n, k, a, b, trans_a=ta, trans_b=tb), want)


def test_the_fp64_product_handles_every_layout():
    rng = np.random.default_rng(2)
    m, n, k = 9, 11, 13
    a = H.bf16_from_f32(rng.normal(0, 1, (m, k)).astype(np.float32))
    b = H.bf16_from_f32(rng.normal(0, 1, (k, n)).astype(np.float32))
    want = H.values(H.BF16, a) @ H.values(H.BF16, b)
    for ta in (False, True):
        for tb in (False, True):
            got, mag = H.gemm_f64(H.BF16, m, n, k, a.T.copy() if ta else a, b.T.copy() if tb else b, trans_a=ta,
                                  trans_b=tb)  # fmt: skip
            assert np.allclose(got, want, rtol=1e-12, atol=1e-12)
            assert np.all(mag >= np.abs(got) - 1e-9)


def test_the_dequant_order_is_stated_and_matters():
    """bf16((f32(acc) * sa) * sb), each product rounded: the oracle gives that, and grouping the scales first (a
    plausible mistake) differs on some element."""
    rng = np.random.default_rng(4)
    acc = rng.integers(-66_000_000, 66_000_000, (512, 512)).astype(np.int32)
    sa = rng.uniform(1e-3, 1e-2, 512).astype(np.float32)
    sb = rng.uniform(1e-3, 1e-2, 512).astype(np.float32)
    got = H.dequant(acc, sa, sb)
    stated = ((acc.astype(np.float32) * sa[:, None]).astype(np.float32) * sb[None, :]).astype(np.float32)
    assert np.array_equal(got, H.bf16_from_f32(stated))
    grouped = (acc.astype(np.float32) * (sa[:, None] * sb[None, :]).astype(np.float32)).astype(np.float32)
    assert not np.array_equal(grouped, stated)  # the f32 values differ ...
    assert not np.array_equal(H.bf16_from_f32(grouped), got)  # ... and some survive the bf16 rounding


def test_gelu_is_the_erf_form():
    o = H.oracle()
    assert o.oracle_gelu(0.0) == 0.0
    for x in (-3.0, -0.5, 0.25, 1.0, 2.5):
        assert o.oracle_gelu(x) == pytest.approx(0.5 * x * (1 + math.erf(x / math.sqrt(2))), rel=1e-15)
    assert o.oracle_gelu(10.0) == pytest.approx(10.0, rel=1e-15)
    assert abs(o.oracle_gelu(-10.0)) < 1e-20
    # the tanh approximation differs by ~1e-4 near x = 1: the test would see a swapped form
    tanh_form = 0.5 * (1 + math.tanh(math.sqrt(2 / math.pi) * (1.0 + 0.044715)))
    assert abs(o.oracle_gelu(1.0) - tanh_form) > 1e-5
