"""The device GELU's arithmetic (cairn_amd/csrc/kernels.hpp, gelu), replayed on the host in f32 step by step with the
constants read from that source: h = Phi(-|x|) = t 2^(q(t) - x^2 log2(e) / 2), t = 1 / (1 + P |x| / sqrt 2), q the
build's degree-8 fit of log2(erfcx(z) (1 + P z)) - 1, then x (1 - h) or x h; against GELU's exact form
0.5 x erfc(-x / sqrt 2) in fp64 (math.erfc has no cancellation, unlike 1 + erf). The device's reciprocal and 2^x are
1-ulp approximations; they are taken as correctly rounded here, so the bounds leave them room. The GPU parity tests
hold the device's own outputs to the contract."""

from __future__ import annotations

import math
import re
from pathlib import Path

import numpy as np
import pytest

SOURCE = Path(__file__).resolve().parents[1] / "cairn_amd" / "csrc" / "kernels.hpp"
f32 = np.float32


def body() -> str:
    return SOURCE.read_text().split("__device__ inline float gelu(float x) {", 1)[1].split("\n}", 1)[0]


def coefficients() -> list[float]:
    """q's coefficients, highest degree first, as the source writes them."""
    b = body()
    first = float(re.search(r"float q = (-?[0-9.]+)f;", b).group(1))
    rest = [float(c) for c in re.findall(r"q = __builtin_fmaf\(q, t, (-?[0-9.]+)f\);", b)]
    return [first, *rest]


def constants() -> tuple[float, float]:
    """P / sqrt 2 (the reciprocal's slope) and log2(e) / 2 (the exponent's), as the source writes them."""
    b = body()
    slope = float(re.search(r"__builtin_fabsf\(x\), (-?[0-9.]+)f, 1.0f\)", b).group(1))
    half_log2e = float(re.search(r"x \* ([0-9.]+)f, q\)", b).group(1))
    return slope, half_log2e


def fma(a, b, c) -> np.float32:
    return f32(np.float64(a) * np.float64(b) + np.float64(c))


def gelu32(x: float, cs: list[float]) -> float:
    slope, half_log2e = constants()
    x = f32(x)
    t = f32(1.0 / np.float64(fma(abs(x), f32(slope), 1.0)))
    q = f32(cs[0])
    for c in cs[1:]:
        q = fma(q, t, f32(c))
    arg = fma(-x, f32(x * f32(half_log2e)), q)
    h = f32(t * f32(np.exp2(np.float64(arg))))
    s = f32(f32(1.0) - h) if x >= 0 else h
    return float(f32(x * s))


def exact(x: float) -> float:
    return 0.5 * x * math.erfc(-x / math.sqrt(2))


def test_the_source_holds_a_degree_8_fit_of_the_stated_function():
    """q(t) against log2(erfcx(z) (1 + P z)) - 1 (scipy's erfcx: exp(z^2) erfc(z) without overflow) on t from
    1 / (1 + P 13.2 / sqrt 2) to 1: within 1e-7 everywhere (the fit's 9.4e-8 with its coefficients in f32). A changed
    or misplaced coefficient moves the curve by far more."""
    from scipy.special import erfcx

    cs = coefficients()
    slope, half_log2e = constants()
    assert len(cs) == 9
    assert f32(half_log2e) == f32(0.5 / math.log(2))
    p = np.float64(f32(slope)) * math.sqrt(2)
    assert abs(p - 0.38) < 1e-7
    t = np.linspace(1 / (1 + p * 13.2 / math.sqrt(2)), 1.0, 200001)
    z = (1 / t - 1) / p
    want = np.log2(erfcx(z) * (1 + p * z)) - 1.0
    held = np.array(cs, dtype=np.float32).astype(np.float64)  # the values the device holds
    assert np.abs(np.polyval(held, t) - want).max() < 1e-7


@pytest.mark.parametrize("limit,bound", [(1.0, 6e-7), (3.0, 1.2e-6), (6.0, 3e-6), (13.0, 1.2e-5)])
def test_relative_error_stays_within_its_bound(limit, bound):
    cs = coefficients()
    xs = np.concatenate([np.linspace(-limit, limit, 40001), np.linspace(-1e-3, 1e-3, 2001)]).astype(np.float32)
    worst = max(abs(gelu32(float(x), cs) - exact(float(x))) / max(abs(exact(float(x))), 1e-38) for x in xs)
    assert worst <= bound, worst


def test_special_values():
    cs = coefficients()
    assert gelu32(0.0, cs) == 0.0 and math.copysign(1.0, gelu32(-0.0, cs)) == -1.0
    assert gelu32(math.inf, cs) == math.inf
    assert math.isnan(gelu32(math.nan, cs))
    assert gelu32(-30.0, cs) == 0.0 and gelu32(30.0, cs) == pytest.approx(30.0, rel=1e-7)
