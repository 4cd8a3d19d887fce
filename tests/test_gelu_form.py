"""The device GELU's arithmetic (cairn_amd/csrc/kernels.hpp, gelu), replayed on the host in f32 step by step with the
coefficients read from that source: the erfc Chebyshev fit of Numerical Recipes (2nd ed., section 6.2, erfcc) in
the branch-free form the kernels use, against GELU's exact form 0.5 x erfc(-x / sqrt 2) in fp64 (math.erfc has no
cancellation, unlike 1 + erf). The device's reciprocal and 2^x are 1-ulp approximations; they are taken as correctly
rounded here, so the bounds leave them room. The GPU parity tests hold the device's own outputs to the contract."""

from __future__ import annotations

import math
import re
from pathlib import Path

import numpy as np
import pytest

SOURCE = Path(__file__).resolve().parents[1] / "cairn_amd" / "csrc" / "kernels.hpp"
f32 = np.float32


def coefficients() -> list[float]:
    body = SOURCE.read_text().split("__device__ inline float gelu(float x) {", 1)[1].split("\n}", 1)[0]
    first = float(re.search(r"float p = (-?[0-9.]+)f;", body).group(1))
    rest = [float(c) for c in re.findall(r"p = __builtin_fmaf\(p, t, (-?[0-9.]+)f\);", body)]
    return [first, *rest]


def fma(a, b, c) -> np.float32:
    return f32(np.float64(a) * np.float64(b) + np.float64(c))


def gelu32(x: float, cs: list[float]) -> float:
    x = f32(x)
    z = f32(abs(x) * f32(0.70710678118654752440))
    t = f32(1.0 / np.float64(fma(0.5, z, 1.0)))
    p = f32(cs[0])
    for c in cs[1:]:
        p = fma(p, t, f32(c))
    arg = fma(-x, f32(f32(0.5) * x), p)
    e = f32(t * f32(np.exp2(np.float64(f32(arg * f32(1.44269504088896340736))))))
    s = f32(2.0) - e if x >= 0 else e
    return float(f32(f32(f32(0.5) * x) * s))


def exact(x: float) -> float:
    return 0.5 * x * math.erfc(-x / math.sqrt(2))


def test_the_source_holds_the_published_fit():
    assert coefficients() == [0.17087277, -0.82215223, 1.48851587, -1.13520398, 0.27886807, -0.18628806, 0.09678418,
                              0.37409196, 1.00002368, -1.26551223]  # fmt: skip


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
