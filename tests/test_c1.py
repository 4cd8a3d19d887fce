"""C1: the f32 GEMM C = A.B on the reference's CPU path at M = N = K = 512, A and B i.i.d.
uniform[-1, 1) from a seeded generator, C from zero, checked against an fp64 host reference at 1e-4 relative error.

The CPU path is the host multiply emitted code calls for host views, cr::tensor::multiply<A> with A = float
(src/cairn/runtime/cairn_tensor.hpp:28-41): for each output its old value, then its k products in increasing p,
every product and sum rounded to f32. It is reached here three ways, which must agree bit for bit: the library's
host entry cf_mma_f32 (include/cairn/cairn_tensor.hpp), the oracle's C restatement, and, where the reference
checkout was built (oracle/_ref), the reference's own header. The error is measured as the reference's error model
states it (src/cairn/compiler/device/tensor.py:10-12), per element against its magnitude:
|got - exact| <= 1e-4 (|c| + sum |a b|); the normwise max |got - exact| / max |exact| is checked beside it.
"""

from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

import helpers as H
from cairn_amd import lib as L

N = 512
SEED = 20261201


def splitmix64(x: np.ndarray) -> np.ndarray:
    """The splitmix64 finalizer of state x + golden gamma (Steele, Lea, Flood 2014), on uint64 arrays."""
    with np.errstate(over="ignore"):
        z = np.asarray(x, dtype=np.uint64) + np.uint64(0x9E3779B97F4A7C15)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def uniform(count: int, seed: int) -> np.ndarray:
    """count values in [-1, 1): the top 24 bits of splitmix64(seed * 2^32 + e) over 2^23, minus 1. Every value is an
    f32 exactly."""
    h = splitmix64(np.arange(count, dtype=np.uint64) + np.uint64(seed) * np.uint64(1 << 32))
    return ((h >> np.uint64(40)).astype(np.float64) / 2.0**23 - 1.0).astype(np.float32)


def test_the_generator_is_uniform_on_minus_one_to_one():
    x = uniform(1 << 16, 3)
    assert x.dtype == np.float32 and x.min() >= -1.0 and x.max() < 1.0
    assert abs(float(x.mean())) < 0.01 and abs(float(x.var()) - 1 / 3) < 0.01
    assert np.array_equal(x, uniform(1 << 16, 3)) and not np.array_equal(x, uniform(1 << 16, 4))


@pytest.fixture(scope="module")
def c1():
    a = uniform(N * N, SEED).reshape(N, N)
    b = uniform(N * N, SEED + 1).reshape(N, N)
    c = np.zeros((N, N), dtype=np.float32)
    lib = L.load()
    lib.cf_mma_f32(N, N, N, c.size, H.ptr(c), a.size, H.ptr(a), b.size, H.ptr(b))
    return a, b, c


def test_c1_is_within_1e_4_of_fp64(c1):
    a, b, got = c1
    exact = a.astype(np.float64) @ b.astype(np.float64)
    mag = np.abs(a.astype(np.float64)) @ np.abs(b.astype(np.float64))
    err = np.abs(got.astype(np.float64) - exact)
    assert np.all(err <= 1e-4 * mag)
    assert float(err.max() / np.abs(exact).max()) <= 1e-4
    # The f32 sum's own bound, much tighter than 1e-4: (k + 1) 2^-24 per rounding, summed.
    assert np.all(err <= (N + 1) * 2.0**-24 * mag)


def test_c1_is_the_host_loop_bit_for_bit(c1):
    a, b, got = c1
    want = np.zeros((N, N), dtype=np.float32)
    assert H.mma(H.F32, N, N, N, want, a, b) == 0
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    if H.REF.exists():  # the reference's own header, compiled from /root/reference (oracle/Makefile)
        ref = C.CDLL(str(H.REF))
        ref.ref_mma_f32.argtypes = [C.c_size_t] * 3 + [C.c_void_p, C.c_size_t] * 3
        theirs = np.zeros((N, N), dtype=np.float32)
        ref.ref_mma_f32(N, N, N, H.ptr(theirs), theirs.size, H.ptr(a), a.size, H.ptr(b), b.size)
        assert np.array_equal(got.view(np.uint32), theirs.view(np.uint32))


def test_a_reordered_sum_would_be_caught(c1):
    """The bit-for-bit check can tell the reference's order from another: summing p downward differs."""
    a, b, got = c1
    rows = slice(0, 4)
    down = np.zeros((4, N), dtype=np.float32)
    for p in range(N - 1, -1, -1):
        down = down + a[rows, p : p + 1] * b[p : p + 1, :]
    assert not np.array_equal(down.view(np.uint32), got[rows].view(np.uint32))
