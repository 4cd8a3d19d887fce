"""The gfx950 kernels against the oracle, through the C ABI (include/cairn_gemm.h).

- The reference's own device shapes (tests/soundness/test_tensor.py:183-222) with its generator: values that are
  multiples of 1/16, so every sum is exact in f32 and the device must equal the host reference loop bit for bit,
  whatever order the matrix cores add in.
- Random bf16/f16 operands on every layout and output type, held to the contract
  |got - exact| <= (k + 1) 2^-22 (|c| + sum |a b|) (src/cairn/compiler/device/tensor.py:10-12), plus the output's
  own rounding for bf16/f16 outputs (half an ulp: 2^-8 |v| for bf16).
- int8 -> int32 bit-exact against exact integer products; the dequant epilogue bit-exact against the oracle's
  stated order bf16((f32(acc) * sa[i]) * sb[j]).
- Bias and ReLU/GELU against fp64 closed forms.
- BASELINE.json's full sizes through the exact fp64 product (BLAS on the host).
"""

from __future__ import annotations

import ctypes as C
import sys

import numpy as np
import pytest
from scipy.special import erf

import helpers as H
from cairn_amd import hip
from cairn_amd import lib as L

pytestmark = pytest.mark.gpu


def say(*what):
    print("[gpu]", *what, flush=True)
    sys.stdout.flush()


def run_gemm(ab_type, c_type, m, n, k, a, b, c_init=None, *, trans_a=False, trans_b=False, accumulate=False,
             act=L.ACT_NONE, bias=None, bias_type=L.F32, row_scale=None, col_scale=None, kernel=0, ldc=0):  # fmt: skip
    """Upload, run one cairn_gemm_run on the null stream, synchronize, download c."""
    out_dtype = {L.F32: np.float32, L.BF16: np.uint16, L.F16: np.uint16, L.I32: np.int32}[c_type]
    ldc = ldc or n
    c_host = np.zeros((m, ldc), dtype=out_dtype) if c_init is None else np.ascontiguousarray(c_init, dtype=out_dtype)
    bufs = [hip.Buffer.of(np.ascontiguousarray(x)) if x is not None else None
            for x in (a, b, c_host, bias, row_scale, col_scale)]  # fmt: skip
    da, db, dc, dbias, drs, dcs = bufs
    d = L.desc(ab_type, c_type, m, n, k, da.ptr if da else None, db.ptr if db else None, dc.ptr,
               trans_a=trans_a, trans_b=trans_b, ldc=ldc, accumulate=accumulate, act=act,
               bias=dbias.ptr if dbias else None, bias_type=bias_type, row_scale=drs.ptr if drs else None,
               col_scale=dcs.ptr if dcs else None, kernel=kernel)  # fmt: skip
    choice = L.select(d)
    say(f"run {L.TYPE_NAMES[ab_type]}->{L.TYPE_NAMES[c_type]} {m}x{n}x{k} ta={trans_a} tb={trans_b} -> {choice['name']}")
    L.run(d)
    hip.synchronize()
    out = dc.download(c_host.shape, out_dtype)
    for x in bufs:
        if x is not None:
            x.close()
    return out, choice


# ------------------------------------------------------------------ the reference's device shapes, exact

DEVICE_SHAPES = [(1, 1, 1, 1), (65, 63, 33, 2), (130, 70, 100, 3), (64, 64, 32, 4), (72, 80, 96, 5), (129, 136, 8, 6),
                 (3, 4, 0, 7)]  # fmt: skip


@pytest.mark.parametrize("name", list(H.FORMATS))
def test_the_reference_device_shapes_equal_the_host_loop_bit_for_bit(name):
    fmt = H.FORMATS[name]
    for m, n, k, seed in DEVICE_SHAPES:
        a = H.encode(fmt, H.device_values(m * k, seed, 2654435761)).reshape(m, k)
        b = H.encode(fmt, H.device_values(k * n, seed * 3, 40503)).reshape(k, n)
        c0 = (H.tile_values(m * n, 99 + seed) / 2).astype(np.float32).reshape(m, n)
        want = c0.copy()
        assert H.mma(fmt, m, n, k, want, a, b) == 0
        got, _ = run_gemm(fmt, L.F32, m, n, k, a, b, c0, accumulate=True)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (name, m, n, k)


def fits(info, m, n, k) -> bool:
    """Whether the kernel `info` names can run an m x n x k problem in its layout (a selector question, no GPU)."""
    ta, tb, t = info["trans_a"], info["trans_b"], info["ab_type"]
    d = L.desc(t, L.I32 if t == L.I8 else L.F32, m, n, k, 1 << 20, 1 << 20, 1 << 20, trans_a=ta, trans_b=tb,
               kernel=info["id"])  # fmt: skip
    return L.load().cairn_gemm_select(C.byref(d), None) == L.OK


def test_the_tile_simulator_shapes_equal_the_host_loop_for_every_kernel():
    """Every tiled kernel (each layout, tile and operand size) on shapes with tails, exact data. A kernel the selector
    refuses for a shape (the one-wave-a-SIMD kernel needs long enough rows) skips it, but runs at least two."""
    for info in L.kernels():
        if info["family"] not in ("mfma", "wave"):
            continue
        ta, tb, t = info["trans_a"], info["trans_b"], info["ab_type"]
        shapes = [(16, 16, 16), (info["tile_m"] + 16, info["tile_n"] + 32, 200), (272, 144, 72), (264, 264, 104),
                  (288, 272, 96)]
        byte = t in (L.I8, L.F8E4M3, L.F8E5M2)
        shapes = [(m, n, (k + 15) // 16 * 16 if byte else k) for m, n, k in shapes]
        shapes = [s for s in shapes if fits(info, *s)]
        assert len(shapes) >= 2, info["name"]
        for m, n, k in shapes:
            if t == L.I8:
                k = (k + 15) // 16 * 16
                av = (H.tile_values(m * k, 7 + m) * 16).astype(np.int8)
                bv = (H.tile_values(k * n, 9 + n) * 16).astype(np.int8)
                a = (av.reshape(k, m) if ta else av.reshape(m, k))
                b = (bv.reshape(n, k) if tb else bv.reshape(k, n))
                got, ch = run_gemm(L.I8, L.I32, m, n, k, a, b, trans_a=ta, trans_b=tb, kernel=info["id"])
                want = H.gemm_i8(m, n, k, a, b, trans_a=ta, trans_b=tb)
                assert np.array_equal(got, want), (info["name"], m, n, k)
            else:
                a = H.encode(t, H.tile_values(m * k, 7 + m)).reshape((k, m) if ta else (m, k))
                b = H.encode(t, H.tile_values(k * n, 9 + n)).reshape((n, k) if tb else (k, n))
                c0 = (H.tile_values(m * n, 5) / 4).astype(np.float32).reshape(m, n)
                got, ch = run_gemm(t, L.F32, m, n, k, a, b, c0, trans_a=ta, trans_b=tb, accumulate=True,
                                   kernel=info["id"])  # fmt: skip
                exact, _ = H.gemm_f64(t, m, n, k, a, b, trans_a=ta, trans_b=tb)
                assert np.array_equal(got, (c0.astype(np.float64) + exact).astype(np.float32)), (info["name"], m, n, k)
            assert ch["kernel"] == info["id"]


def test_every_ring_kernel_rounds_its_own_f32_result_to_bf16():
    """The plain bf16 output (no epilogue) of each LDS-ring kernel is the nearest-even rounding of what the same
    kernel computes in f32: the fast store path and the general one agree bit for bit."""
    rng = np.random.default_rng(77)
    for info in L.kernels():
        if info["family"] != "wave" or info["ab_type"] != L.BF16:
            continue
        ta, tb = info["trans_a"], info["trans_b"]
        m, n, k = info["tile_m"] + 40, info["tile_n"] + 24, 136
        a = H.normal_bf16(rng, (k, m) if ta else (m, k), 1.0)
        b = H.normal_bf16(rng, (n, k) if tb else (k, n), 1.0)
        f32, _ = run_gemm(L.BF16, L.F32, m, n, k, a, b, trans_a=ta, trans_b=tb, kernel=info["id"])
        b16, _ = run_gemm(L.BF16, L.BF16, m, n, k, a, b, trans_a=ta, trans_b=tb, kernel=info["id"])
        assert np.array_equal(b16, H.bf16_from_f32(f32)), info["name"]


@pytest.mark.parametrize("act", [L.ACT_NONE, L.ACT_RELU])
def test_every_ring_kernel_applies_the_epilogue_in_its_stated_order(act):
    """Row and column scales, a bias and an activation on every LDS-ring kernel of every operand type, bf16 out:
    whole tiles take the LDS-staged store, edge tiles the checked one, and both equal the stated steps applied in f32
    to what the same kernel computes without them: bf16(act((f32(acc) * rs[i]) * cs[j] + bias[j]))."""
    rng = np.random.default_rng(78 + act)
    ran = 0
    for info in L.kernels():
        if info["family"] != "wave":
            continue
        ta, tb, t = info["trans_a"], info["trans_b"], info["ab_type"]
        m, n, k = info["tile_m"] + 40, info["tile_n"] + 24, 144
        if not fits(info, m, n, k):
            continue
        if t == L.I8:
            a = rng.integers(-127, 128, (k, m) if ta else (m, k), dtype=np.int8)
            b = rng.integers(-127, 128, (n, k) if tb else (k, n), dtype=np.int8)
        elif t in (L.F8E4M3, L.F8E5M2):
            a = H.encode(t, rng.standard_normal(m * k).clip(-8, 8)).reshape((k, m) if ta else (m, k))
            b = H.encode(t, rng.standard_normal(k * n).clip(-8, 8)).reshape((n, k) if tb else (k, n))
        else:
            a = H.normal_bf16(rng, (k, m) if ta else (m, k), 1.0)
            b = H.normal_bf16(rng, (n, k) if tb else (k, n), 1.0)
        rs = rng.uniform(0.25, 2.0, m).astype(np.float32)
        cs = rng.uniform(0.25, 2.0, n).astype(np.float32)
        bias = H.normal_bf16(rng, (n,), 4.0)
        raw, _ = run_gemm(t, L.I32 if t == L.I8 else L.F32, m, n, k, a, b, trans_a=ta, trans_b=tb, kernel=info["id"])
        got, _ = run_gemm(t, L.BF16, m, n, k, a, b, trans_a=ta, trans_b=tb, row_scale=rs, col_scale=cs, bias=bias,
                          bias_type=L.BF16, act=act, kernel=info["id"])  # fmt: skip
        v = raw.astype(np.float32) * rs[:, None]
        v = v * cs[None, :]
        v = v + H.f32_from_bf16(bias)[None, :]
        if act == L.ACT_RELU:
            v = np.where(v < 0, np.float32(0), v)
        assert np.array_equal(got, H.bf16_from_f32(v)), info["name"]
        ran += 1
    assert ran >= 10


@pytest.mark.parametrize("name", ["cairn_wave_bf16_nn_256x256"])
def test_bf16_outputs_round_ties_to_even_keep_subnormals_and_overflow(name):
    """Outputs exact in f32 that sit on bf16 rounding ties: near 1 (c = b0 +- 2^-8), among the subnormals
    (c = 2^-127 b0, spacing 2^-133 against f32's 2^-149) and at the top (c = 2^127 (b0 + 2^-8), whose last tie rounds
    to infinity). The bf16 output must be the f32 output narrowed (nearest even, the reference's narrow<bf16>)."""
    m, n, k = 256, 256, 32
    rows = np.arange(m) % 4
    a = np.zeros((m, k), dtype=np.float64)
    a[:, 0] = np.select([rows == 0, rows == 1, rows == 2, rows == 3], [1.0, 1.0, 2.0**-127, 2.0**127])
    a[:, 1] = np.select([rows == 0, rows == 1, rows == 2, rows == 3], [2.0**-8, -(2.0**-8), 0.0, 2.0**119])
    b = np.zeros((k, n), dtype=np.float64)
    b[0, :] = 1.0 + (np.arange(n) % 128) / 128.0
    b[1, :] = 1.0
    a16, b16 = H.encode(L.BF16, a.ravel()).reshape(m, k), H.encode(L.BF16, b.ravel()).reshape(k, n)
    assert np.array_equal(H.values(L.BF16, a16), a) and np.array_equal(H.values(L.BF16, b16), b)  # exact operands
    kernel = L.kernel_named(name)
    f32, ch = run_gemm(L.BF16, L.F32, m, n, k, a16, b16, kernel=kernel)
    assert ch["name"] == name
    exact = a @ b
    assert np.array_equal(f32.astype(np.float64), exact)  # every output exact in f32
    out, _ = run_gemm(L.BF16, L.BF16, m, n, k, a16, b16, kernel=kernel)
    assert np.array_equal(out, H.bf16_from_f32(f32))
    assert np.isinf(H.f32_from_bf16(out[3::4, 127])).all()  # 2^127 (2 - 2^-7 + 2^-8) rounds up to infinity
    assert (H.f32_from_bf16(out[2::4, :]) <= 2.0**-126).all()  # the subnormal rows reach at most the least normal


# ------------------------------------------------------------------ random operands: the contract

LAYOUTS = [(False, False), (False, True), (True, False), (True, True)]


@pytest.mark.parametrize("trans_a,trans_b", LAYOUTS)
@pytest.mark.parametrize("fmt", [L.BF16, L.F16])
def test_random_operands_keep_the_contract_on_every_layout(fmt, trans_a, trans_b):
    rng = np.random.default_rng(20261201 + 2 * trans_a + trans_b)
    for m, n, k in [(256, 256, 128), (520, 264, 200), (72, 1032, 1000)]:
        av = rng.normal(0, 1, (k, m) if trans_a else (m, k)).astype(np.float32)
        bv = rng.normal(0, 1, (n, k) if trans_b else (k, n)).astype(np.float32)
        a = H.bf16_from_f32(av) if fmt == L.BF16 else av.astype(np.float16).view(np.uint16)
        b = H.bf16_from_f32(bv) if fmt == L.BF16 else bv.astype(np.float16).view(np.uint16)
        A = H.values(fmt, a)
        B = H.values(fmt, b)
        A = A.T if trans_a else A
        B = B.T if trans_b else B
        exact, mag = H.exact_product(A, B)
        c0 = rng.uniform(-4, 4, (m, n)).astype(np.float32)
        got, ch = run_gemm(fmt, L.F32, m, n, k, a, b, c0, trans_a=trans_a, trans_b=trans_b, accumulate=True)
        assert ch["family"] in ("mfma", "wave")
        assert H.outside(got, c0 + exact, H.bound(k, c0, mag)) == 0
        # bf16 output: the contract plus half an ulp of the output format.
        got16, _ = run_gemm(fmt, L.BF16, m, n, k, a, b, trans_a=trans_a, trans_b=trans_b)
        v = H.f32_from_bf16(got16)
        room = H.bound(k, np.zeros_like(c0), mag) + 2.0**-8 * np.abs(exact) * 1.01
        assert H.outside(v, exact, room) == 0


def f8_patterns(rng, fmt: int, shape) -> np.ndarray:
    """Every finite pattern of the 8-bit float at random, subnormals and the largest values included."""
    p = rng.integers(0, 256, shape, dtype=np.uint8)
    bad = ~np.isfinite(H.values(fmt, p))
    while bad.any():
        p[bad] = rng.integers(0, 256, int(bad.sum()), dtype=np.uint8)
        bad = ~np.isfinite(H.values(fmt, p))
    return p


@pytest.mark.parametrize("trans_a,trans_b", LAYOUTS)
@pytest.mark.parametrize("fmt", [L.F8E4M3, L.F8E5M2])
def test_fp8_keeps_the_contract_on_every_layout(fmt, trans_a, trans_b):
    """The 8-bit floats as the selector runs them (widened to f16 on their way into LDS, the f16 matrix core): random
    patterns over the whole range, short k (where one large product and many small ones share a group of the matrix
    core's adds) and long, products exact, each sum within the contract of its exact value."""
    rng = np.random.default_rng(8 + 4 * fmt + 2 * trans_a + trans_b)
    for m, n, k in [(512, 768, 1024), (1536, 1040, 272), (264, 136, 16), (136, 264, 72)]:
        a = f8_patterns(rng, fmt, (k, m) if trans_a else (m, k))
        b = f8_patterns(rng, fmt, (n, k) if trans_b else (k, n))
        A, B = H.values(fmt, a), H.values(fmt, b)
        exact, mag = H.exact_product(A.T if trans_a else A, B.T if trans_b else B)
        c0 = rng.uniform(-4, 4, (m, n)).astype(np.float32)
        got, ch = run_gemm(fmt, L.F32, m, n, k, a, b, c0, trans_a=trans_a, trans_b=trans_b, accumulate=True)
        assert ch["name"].startswith("cairn_mfma_f8"), ch["name"]
        assert H.outside(got, c0 + exact, H.bound(k, c0, mag)) == 0, (m, n, k)


@pytest.mark.parametrize("trans_a,trans_b", LAYOUTS)
@pytest.mark.parametrize("fmt", [L.F8E4M3, L.F8E5M2])
def test_every_pattern_pair_of_the_8_bit_floats_multiplies_exactly(fmt, trans_a, trans_b):
    """a's column 0 holds each of the 256 patterns once, b's row 0 each once (the rest of k zero): c[i, j] is the
    product of patterns i and j, exact in f32 (its sign too, where it is not zero), NaN where either is NaN or an
    infinity meets zero, so every pattern widens to its own value in both operands' loads (K- and M/N-contiguous)."""
    m = n = 256
    k = 8
    pats = np.arange(256, dtype=np.uint8)
    zero = np.uint8(0)
    a = np.full((m, k), zero, dtype=np.uint8)
    a[:, 0] = pats
    b = np.full((k, n), zero, dtype=np.uint8)
    b[0, :] = pats[::-1]
    v = H.values(fmt, pats)
    with np.errstate(invalid="ignore", over="ignore"):
        want = v[:, None] * v[::-1][None, :]
    got, ch = run_gemm(fmt, L.F32, m, n, k, np.ascontiguousarray(a.T) if trans_a else a,
                       np.ascontiguousarray(b.T) if trans_b else b, trans_a=trans_a, trans_b=trans_b)  # fmt: skip
    assert ch["name"].startswith("cairn_mfma_f8"), ch["name"]
    g = got.astype(np.float64)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(g), nan)
    assert np.array_equal(g[~nan], want[~nan])
    # Signs of the nonzero results (a zero product's sign is lost to the +0 products of the rest of k: -0 + +0 = +0).
    live = ~nan & (want != 0)
    assert np.array_equal(np.signbit(g[live]), np.signbit(want[live]))


@pytest.mark.parametrize("fmt", [L.F8E4M3, L.F8E5M2])
def test_fp8_keeps_products_far_below_the_largest_in_its_group(fmt):
    """One product of 2^8 and fifteen of 2^-6 in each 16 of k (2^7 and 2^-7 in odd columns): their sum is exact in
    f32, and the selector's path returns it bit for bit. The 8-bit float matrix core (the ring's wave8 kernels, which
    run only where named) adds such a group with a narrower alignment and loses part of the small terms."""
    small = 2.0**-6
    m, n, k = 256, 256, 64
    A = np.full((m, k), small, dtype=np.float64)
    A[:, ::16] = 16.0
    B = np.ones((k, n), dtype=np.float64)
    B[::16, :] = 16.0
    B[:, 1::2] *= 0.5
    a, b = H.encode(fmt, A.ravel()).reshape(m, k), H.encode(fmt, B.ravel()).reshape(k, n)
    assert np.array_equal(H.values(fmt, a), A) and np.array_equal(H.values(fmt, b), B)
    exact = A @ B
    assert np.array_equal(exact.astype(np.float32).astype(np.float64), exact)
    got, ch = run_gemm(fmt, L.F32, m, n, k, a, b)
    assert ch["name"].startswith("cairn_mfma_f8"), ch["name"]
    assert np.array_equal(got.astype(np.float64), exact)


@pytest.mark.parametrize("fmt", [L.F8E4M3, L.F8E5M2])
def test_the_fp8_matrix_core_kernels_at_long_k(fmt):
    """The ring's 8-bit float kernels (v_mfma_f32_32x32x64_f8f6f4, not widened; run where named), every layout, at
    k = 1024 on random patterns: there the contract's room, (k + 1) 2^-22 sum |a b|, holds what their grouped adds
    lose. (At short k it does not: the selector's path widens instead.)"""
    rng = np.random.default_rng(18 + fmt)
    m, n, k = 512, 768, 1024
    for ta, tb in LAYOUTS:
        lay = ("t" if ta else "n") + ("t" if tb else "n")
        a = f8_patterns(rng, fmt, (k, m) if ta else (m, k))
        b = f8_patterns(rng, fmt, (n, k) if tb else (k, n))
        A, B = H.values(fmt, a), H.values(fmt, b)
        exact, mag = H.exact_product(A.T if ta else A, B.T if tb else B)
        c0 = rng.uniform(-4, 4, (m, n)).astype(np.float32)
        name = f"cairn_wave_{L.TYPE_NAMES[fmt].lower()}_{lay}_256x256"
        got, ch = run_gemm(fmt, L.F32, m, n, k, a, b, c0, trans_a=ta, trans_b=tb, accumulate=True,
                           kernel=L.kernel_named(name))  # fmt: skip
        assert ch["name"] == name
        assert H.outside(got, c0 + exact, H.bound(k, c0, mag)) == 0, name


def test_two_runs_give_the_same_bits():
    rng = np.random.default_rng(5)
    m, n, k = 1024, 768, 2048
    a = H.normal_bf16(rng, (m, k), 1.0)
    b = H.normal_bf16(rng, (k, n), 1.0)
    first, _ = run_gemm(L.BF16, L.F32, m, n, k, a, b)
    second, _ = run_gemm(L.BF16, L.F32, m, n, k, a, b)
    assert np.array_equal(first.view(np.uint32), second.view(np.uint32))


# ------------------------------------------------------------------ int8


@pytest.mark.parametrize("trans_a,trans_b", LAYOUTS)
def test_int8_accumulators_are_bit_exact(trans_a, trans_b):
    rng = np.random.default_rng(8 + 2 * trans_a + trans_b)
    for m, n, k in [(200, 136, 80), (512, 520, 1024)]:
        a = rng.integers(-127, 128, (k, m) if trans_a else (m, k), dtype=np.int8)
        b = rng.integers(-127, 128, (n, k) if trans_b else (k, n), dtype=np.int8)
        got, ch = run_gemm(L.I8, L.I32, m, n, k, a, b, trans_a=trans_a, trans_b=trans_b)
        A = a.T if trans_a else a
        B = b.T if trans_b else b
        want = (A.astype(np.float64) @ B.astype(np.float64)).astype(np.int64)  # exact: every sum is below 2^53
        assert np.array_equal(got.astype(np.int64), want), (m, n, k)


def test_int8_extremes_do_not_overflow():
    """All -128 against all -128 with k = 4096: 4096 * 16384 = 2^26, inside int32."""
    m, n, k = 64, 64, 4096
    a = np.full((m, k), -128, dtype=np.int8)
    b = np.full((k, n), -128, dtype=np.int8)
    got, _ = run_gemm(L.I8, L.I32, m, n, k, a, b)
    assert np.all(got == 4096 * 16384)


def test_the_dequant_epilogue_is_bit_exact():
    rng = np.random.default_rng(44)
    m, n, k = 384, 264, 512
    a = rng.integers(-127, 128, (m, k), dtype=np.int8)
    b = rng.integers(-127, 128, (k, n), dtype=np.int8)
    sa = rng.uniform(1e-3, 1e-2, m).astype(np.float32)
    sb = rng.uniform(1e-3, 1e-2, n).astype(np.float32)
    got, _ = run_gemm(L.I8, L.BF16, m, n, k, a, b, row_scale=sa, col_scale=sb)
    acc = H.gemm_i8(m, n, k, a, b)
    assert np.array_equal(got, H.dequant(acc, sa, sb))


# ------------------------------------------------------------------ epilogues


@pytest.mark.parametrize("act", [L.ACT_NONE, L.ACT_RELU, L.ACT_GELU])
def test_bias_and_activation_match_the_closed_form(act):
    rng = np.random.default_rng(3 + act)
    m, n, k = 264, 392, 256
    a = H.normal_bf16(rng, (m, k), 0.5)
    b = H.normal_bf16(rng, (k, n), 0.5)
    bias = H.normal_bf16(rng, (n,), 0.5)
    exact, mag = H.exact_product(H.values(L.BF16, a), H.values(L.BF16, b))
    pre = exact + H.values(L.BF16, bias)[None, :]
    if act == L.ACT_RELU:
        want = np.maximum(pre, 0)
    elif act == L.ACT_GELU:
        o = H.oracle()
        want = np.vectorize(o.oracle_gelu)(pre)
    else:
        want = pre
    got, _ = run_gemm(L.BF16, L.BF16, m, n, k, a, b, bias=bias, bias_type=L.BF16, act=act)
    v = H.f32_from_bf16(got).astype(np.float64)
    # The accumulator's contract error passes through the activation (slope <= 1.13 for GELU), then f32 erf's few
    # ulps, then the bf16 output rounding.
    room = 1.2 * H.bound(k, np.zeros(1), mag + np.abs(pre)) + 2.0**-8 * np.abs(want) * 1.01 + 1e-6
    assert H.outside(v, want, room) == 0


# ------------------------------------------------------------------ skinny decode shapes


@pytest.mark.parametrize("m", [1, 4, 8, 16])
def test_skinny_decode_shapes_keep_the_contract(m):
    rng = np.random.default_rng(100 + m)
    n, k = 14336, 4096
    a = H.normal_bf16(rng, (m, k), 1.0)
    b = H.normal_bf16(rng, (n, k), 1.0 / 64)  # stored n x k: K-contiguous
    got, ch = run_gemm(L.BF16, L.BF16, m, n, k, a, b, trans_b=True)
    assert ch["family"] == "skinny"
    exact, mag = H.exact_product(H.values(L.BF16, a), H.values(L.BF16, b).T)
    v = H.f32_from_bf16(got)
    room = H.bound(k, np.zeros(1), mag) + 2.0**-8 * np.abs(exact) * 1.01
    assert H.outside(v, exact, room) == 0


# m >= 2 with n = 8193 .. 16384, and m > 4 from n = 7681, take the half-height ring (32 rows of b a workgroup at most,
# n over 512 workgroups, 512-byte stages); other m > 4 with n >= 4096 the ring form with 256-byte stages (32 columns a
# workgroup below n = 8192, 64 above, two workgroups a CU past 256 of them), m = 1 with n >= 2048 and k <= 4096 the row-streaming one (whole rows
# of b a wave, dealt evenly: a wave's share differs from the next one's by at most a row), m = 2 .. 4 with n >= 2048 the streaming MFMA form (16 rows of b a wave; whole groups of 8 steps, then
# single steps, the last one partial), the rest the register form: tails in each.
@pytest.mark.parametrize("m,n,k", [(1, 8, 8), (3, 100, 72), (16, 33, 4104), (7, 14336, 24), (5, 200, 4160),
                                   (2, 72, 1000), (3, 8200, 4104), (16, 9000, 520), (1, 8192, 8), (9, 8257, 1032),
                                   (1, 4100, 4096), (1, 3000, 1000), (1, 20000, 264), (1, 2048, 4088), (5, 8256, 4096),
                                   (2, 2048, 8), (4, 3001, 1000), (2, 70001, 40), (4, 2050, 520), (3, 14336, 4096),
                                   (8, 4096, 1000), (11, 6150, 264), (6, 20003, 520), (16, 28672, 136),
                                   (5, 4095, 256), (1, 14336, 4096), (1, 12289, 1000), (1, 12288, 520),
                                   (2, 11008, 4104), (4, 10241, 4096), (9, 12289, 24), (16, 16384, 520),
                                   (5, 14336, 1000), (6, 8000, 1000), (3, 8193, 264), (12, 16384, 4096),
                                   (2, 14336, 4096), (2, 4100, 1000), (2, 16384, 264), (2, 8192, 4096)])
def test_skinny_tails_keep_the_contract(m, n, k):
    rng = np.random.default_rng(m * n + k)
    a = H.normal_bf16(rng, (m, k), 1.0)
    b = H.normal_bf16(rng, (n, k), 1.0)
    c0 = rng.uniform(-4, 4, (m, n)).astype(np.float32)
    got, ch = run_gemm(L.BF16, L.F32, m, n, k, a, b, c0, trans_b=True, accumulate=True)
    assert ch["family"] == "skinny"
    exact, mag = H.exact_product(H.values(L.BF16, a), H.values(L.BF16, b).T)
    assert H.outside(got, c0 + exact, H.bound(k, c0, mag)) == 0


@pytest.mark.parametrize("m,n", [(1, 2048), (1, 4100), (1, 12289), (1, 14336), (2, 4100), (2, 14336)])
def test_the_row_streaming_form_rounds_its_own_f32_result_to_each_output_type(m, n):
    """m = 1 and 2 (the row-streaming form, an instance per output type): bf16 and f16 outputs without an epilogue
    are, bit for bit, the same form's f32 result rounded to nearest even."""
    rng = np.random.default_rng(n + m)
    k = 1000
    a = H.normal_bf16(rng, (m, k), 1.0)
    b = H.normal_bf16(rng, (n, k), 1.0)
    raw, ch = run_gemm(L.BF16, L.F32, m, n, k, a, b, trans_b=True)
    assert ch["family"] == "skinny"
    got_bf16, _ = run_gemm(L.BF16, L.BF16, m, n, k, a, b, trans_b=True)
    got_f16, _ = run_gemm(L.BF16, L.F16, m, n, k, a, b, trans_b=True)
    assert np.array_equal(got_bf16, H.bf16_from_f32(raw))
    assert np.array_equal(got_f16, H.narrow_array(H.F16, raw))


@pytest.mark.parametrize("act", [L.ACT_NONE, L.ACT_RELU])
def test_every_skinny_form_applies_the_epilogue_in_its_stated_order(act):
    """Row and column scales, a bf16 bias and an activation on each skinny form (the ring at both of its stage
    sizes), bf16 out: equal, bit for bit, to the stated steps applied in f32 to what the same form computes without
    them: bf16(act((f32(acc) * rs[i]) * cs[j] + bias[j]))."""
    rng = np.random.default_rng(31 + act)
    # rows (m = 1, 2), stream, ring (256-byte stages), register, half-height ring (512-byte stages)
    for m, n, k in [(1, 4100, 1024), (2, 8192, 1000), (3, 4100, 1000), (6, 6000, 512), (3, 200, 256), (6, 14336, 520)]:
        a = H.normal_bf16(rng, (m, k), 1.0)
        b = H.normal_bf16(rng, (n, k), 1.0)
        rs = rng.uniform(0.25, 2.0, m).astype(np.float32)
        cs = rng.uniform(0.25, 2.0, n).astype(np.float32)
        bias = H.normal_bf16(rng, (n,), 4.0)
        raw, ch = run_gemm(L.BF16, L.F32, m, n, k, a, b, trans_b=True)
        assert ch["family"] == "skinny"
        got, _ = run_gemm(L.BF16, L.BF16, m, n, k, a, b, trans_b=True, row_scale=rs, col_scale=cs, bias=bias,
                          bias_type=L.BF16, act=act)  # fmt: skip
        v = raw.astype(np.float32) * rs[:, None]
        v = v * cs[None, :]
        v = v + H.f32_from_bf16(bias)[None, :]
        if act == L.ACT_RELU:
            v = np.where(v < 0, np.float32(0), v)
        assert np.array_equal(got, H.bf16_from_f32(v)), (m, n, k)


# ------------------------------------------------------------------ BASELINE.json's full sizes


def test_bf16_4096_cubed_keeps_the_contract():
    rng = np.random.default_rng(4096)
    n = 4096
    a = H.normal_bf16(rng, (n, n), 1 / 64)
    b = H.normal_bf16(rng, (n, n), 1 / 64)
    got, ch = run_gemm(L.BF16, L.BF16, n, n, n, a, b)
    say("4096^3 ran on", ch["name"])
    exact, mag = H.exact_product(H.values(L.BF16, a), H.values(L.BF16, b))
    v = H.f32_from_bf16(got)
    room = H.bound(n, np.zeros(1), mag) + 2.0**-8 * np.abs(exact) * 1.01
    assert H.outside(v, exact, room) == 0
    # BASELINE's metric: max |got - ref| / (sum |a b|) <= 1e-2.
    assert float(np.max(np.abs(v - exact) / mag)) <= 1e-2


def test_int8_4096_cubed_is_bit_exact():
    rng = np.random.default_rng(8)
    n = 4096
    a = rng.integers(-127, 128, (n, n), dtype=np.int8)
    b = rng.integers(-127, 128, (n, n), dtype=np.int8)
    got, _ = run_gemm(L.I8, L.I32, n, n, n, a, b)
    want = a.astype(np.float64) @ b.astype(np.float64)
    assert np.array_equal(got.astype(np.float64), want)


def test_the_mlp_layer_at_full_size_keeps_the_contract():
    """C3 at BASELINE.json's size, on the GPU in full: the forward Y = GELU(X W + b) (NN, bias and GELU fused, bf16
    out), dX = dY W^T (NT) and dW = X^T dY (TN), with X 8192 x 4096, W 4096 x 11008, dY 8192 x 11008. Checked
    against the exact fp64 product on a sample of 256 output rows of each (the host's BLAS): each output within
    the contract's bound plus its bf16 rounding, GELU's slope (<= 1.13) carried through."""
    rng = np.random.default_rng(3)
    m, k, n = 8192, 4096, 11008
    x = H.normal_bf16(rng, (m, k), 1.0)
    w = H.normal_bf16(rng, (k, n), 0.02)
    bias = H.normal_bf16(rng, (n,), 0.02)
    dy = H.normal_bf16(rng, (m, n), 1.0)
    xv, wv, dyv = H.values(L.BF16, x), H.values(L.BF16, w), H.values(L.BF16, dy)
    rows = np.sort(rng.choice(m, 256, replace=False))
    o = H.oracle()

    y, ch = run_gemm(L.BF16, L.BF16, m, n, k, x, w, bias=bias, bias_type=L.BF16, act=L.ACT_GELU)
    say("mlp forward ran on", ch["name"])
    exact, mag = H.exact_product(xv[rows], wv)
    pre = exact + H.values(L.BF16, bias)[None, :]
    want = 0.5 * pre * (1.0 + erf(pre / np.sqrt(2.0)))  # the oracle's GELU (oracle_gelu), vectorized
    assert abs(float(want[0, 0]) - o.oracle_gelu(float(pre[0, 0]))) <= 1e-15 * max(1.0, abs(float(want[0, 0])))
    room = 1.2 * H.bound(k, np.zeros(1), mag + np.abs(pre)) + 2.0**-8 * np.abs(want) * 1.01 + 1e-6
    assert H.outside(H.f32_from_bf16(y[rows]), want, room) == 0

    dx, ch = run_gemm(L.BF16, L.BF16, m, k, n, dy, w, trans_b=True)
    say("mlp dX ran on", ch["name"])
    exact, mag = H.exact_product(dyv[rows], wv.T)
    room = H.bound(n, np.zeros(1), mag) + 2.0**-8 * np.abs(exact) * 1.01
    assert H.outside(H.f32_from_bf16(dx[rows]), exact, room) == 0

    dw, ch = run_gemm(L.BF16, L.BF16, k, n, m, x, dy, trans_a=True)
    say("mlp dW ran on", ch["name"])
    wrows = np.sort(rng.choice(k, 256, replace=False))
    exact, mag = H.exact_product(xv[:, wrows].T, dyv)
    room = H.bound(m, np.zeros(1), mag) + 2.0**-8 * np.abs(exact) * 1.01
    assert H.outside(H.f32_from_bf16(dw[wrows]), exact, room) == 0


# ------------------------------------------------------------------ padded leading dimensions


def padded(x: np.ndarray, ld: int, fill=0) -> np.ndarray:
    """x (rows x cols) stored with `ld` elements a row; the padding holds `fill`."""
    out = np.full((x.shape[0], ld), fill, dtype=x.dtype)
    out[:, : x.shape[1]] = x
    return out


@pytest.mark.parametrize("ldc_pad", [4, 8])
def test_padded_leading_dimensions_on_every_tiled_kernel(ldc_pad):
    """Every tiled kernel with lda and ldb 16 elements past their rows and ldc = n + 4 (bf16 rows of c on 8 bytes:
    the checked 8-byte stores) or n + 8 (on 16 bytes: the LDS-staged 16-byte stores), on whole tiles and on tails.
    Exact data, so a bf16 output is the exact sum rounded once, and int8 is exact both as int32 and through unit
    dequant scales into bf16; the padding of c keeps its bytes."""
    ran = 0
    for info in L.kernels():
        if info["family"] not in ("mfma", "wave"):
            continue
        ta, tb, t = info["trans_a"], info["trans_b"], info["ab_type"]
        for m, n, k in [(2 * info["tile_m"], 2 * info["tile_n"], 256), (info["tile_m"] + 40, info["tile_n"] + 24, 208)]:
            arow, brow = (m if ta else k), (k if tb else n)
            lda, ldb, ldc = arow + 16, brow + 16, n + ldc_pad
            d = L.desc(t, L.I32 if t == L.I8 else L.BF16, m, n, k, 1 << 20, 1 << 20, 1 << 20, trans_a=ta, trans_b=tb,
                       lda=lda, ldb=ldb, ldc=ldc, kernel=info["id"])  # fmt: skip
            if L.load().cairn_gemm_select(C.byref(d), None) != L.OK:
                continue
            if t == L.I8:
                a = (H.tile_values(m * k, 3 + m) * 16).astype(np.int8).reshape((k, m) if ta else (m, k))
                b = (H.tile_values(k * n, 5 + n) * 16).astype(np.int8).reshape((n, k) if tb else (k, n))
                exact = H.gemm_i8(m, n, k, a, b, trans_a=ta, trans_b=tb).astype(np.float64)
                outs = [(L.I32, np.int32, 0x5A5A5A5A), (L.BF16, np.uint16, 0x7A7A)]
            else:
                a = H.encode(t, H.tile_values(m * k, 3 + m)).reshape((k, m) if ta else (m, k))
                b = H.encode(t, H.tile_values(k * n, 5 + n)).reshape((n, k) if tb else (k, n))
                exact, _ = H.gemm_f64(t, m, n, k, a, b, trans_a=ta, trans_b=tb)
                outs = [(L.BF16, np.uint16, 0x7A7A)]
            ap, bp = padded(a, lda), padded(b, ldb)
            for out_type, out_dtype, sentinel in outs:
                say(f"padded {info['name']} {m}x{n}x{k} lda {lda} ldb {ldb} ldc {ldc} -> {L.TYPE_NAMES[out_type]}")
                c_host = np.full((m, ldc), sentinel, dtype=out_dtype)
                ones_m, ones_n = np.ones(m, np.float32), np.ones(n, np.float32)
                scaled = t == L.I8 and out_type == L.BF16
                bufs = [hip.Buffer.of(x) for x in (ap, bp, c_host, ones_m, ones_n)]
                d = L.desc(t, out_type, m, n, k, bufs[0].ptr, bufs[1].ptr, bufs[2].ptr, trans_a=ta, trans_b=tb,
                           lda=lda, ldb=ldb, ldc=ldc, kernel=info["id"], row_scale=bufs[3].ptr if scaled else None,
                           col_scale=bufs[4].ptr if scaled else None)  # fmt: skip
                L.run(d)
                hip.synchronize()
                got = bufs[2].download(c_host.shape, out_dtype)
                for x in bufs:
                    x.close()
                if out_type == L.I32:
                    assert np.array_equal(got[:, :n].astype(np.float64), exact), (info["name"], m, n, k, ldc)
                else:
                    want = H.bf16_from_f32(exact.astype(np.float32))
                    assert np.array_equal(got[:, :n], want), (info["name"], m, n, k, ldc)
                assert np.all(got[:, n:] == out_dtype(sentinel)), (info["name"], "wrote into the padding of c")
                ran += 1
    assert ran >= 20


def test_w8a8_with_its_fused_dequant_at_4096_cubed():
    """C4 whole: int8 4096^3 with per-row and per-column f32 scales U[1e-3, 1e-2] fused into the epilogue, bf16 out.
    512 sampled rows against the oracle's dequant of the exact int32 sums (bf16((f32(acc) * sa[i]) * sb[j])), bit
    for bit."""
    rng = np.random.default_rng(44096)
    n = 4096
    a = rng.integers(-127, 128, (n, n), dtype=np.int8)
    b = rng.integers(-127, 128, (n, n), dtype=np.int8)
    sa = rng.uniform(1e-3, 1e-2, n).astype(np.float32)
    sb = rng.uniform(1e-3, 1e-2, n).astype(np.float32)
    got, ch = run_gemm(L.I8, L.BF16, n, n, n, a, b, row_scale=sa, col_scale=sb)
    say("W8A8 4096^3 ran on", ch["name"])
    rows = np.sort(rng.choice(n, 512, replace=False))
    acc = (a[rows].astype(np.float64) @ b.astype(np.float64)).astype(np.int32)  # exact: |sums| < 2^26
    assert np.array_equal(got[rows], H.dequant(acc, sa[rows], sb)), "dequant differs from the oracle's order"
