"""The device quantize (cairn_quantize_run) against the oracle's row contract, bit for bit, through the C ABI.

Every input type (f32, f16, bf16) into every output type (int8, E4M3, E5M2) under every scale mode, on shapes that
take each path of the kernel: vector chunks and the element-wise path (k or the leading dimension not a multiple of
8), one pass and two (rows longer than the 8192 elements a workgroup holds). The rows hold what stresses the
arithmetic: exact ties and values a few units from them (the f32 shortcut must hand these to the exact path),
saturation, subnormals, zeros of both signs, NaN and infinity, and scales outside the shortcut's range. Then the
W8A8 chain the kernel exists for: bf16 activations and weights quantized on the device, multiplied by the int8
kernel with their scales, equal to the oracle's chain.
"""

from __future__ import annotations

import sys

import numpy as np
import pytest

import helpers as H
from cairn_amd import hip
from cairn_amd import lib as L

pytestmark = pytest.mark.gpu

RANGE = {L.I8: 127.0, L.F8E4M3: 448.0, L.F8E5M2: 57344.0}
X_TYPES = {"f32": L.F32, "f16": L.F16, "bf16": L.BF16}
Q_TYPES = {"i8": L.I8, "e4m3": L.F8E4M3, "e5m2": L.F8E5M2}
MODES = {"absmax": L.SCALE_ROW_ABSMAX, "row": L.SCALE_ROW, "tensor": L.SCALE_TENSOR}


def say(*what):
    print("[gpu]", *what, flush=True)
    sys.stdout.flush()


def patterns(x_type: int, x: np.ndarray) -> np.ndarray:
    """f32 values into the input type's storage (bf16/f16 patterns, nearest even)."""
    if x_type == L.F32:
        return np.ascontiguousarray(x, dtype=np.float32)
    if x_type == L.BF16:
        return H.bf16_from_f32(x)
    with np.errstate(over="ignore"):
        return np.ascontiguousarray(x.astype(np.float16).view(np.uint16))


def run_quantize(x_type, q_type, mode, xs: np.ndarray, k: int, scale=None, ldq: int = 0):
    """Upload xs (m rows of ldx elements), quantize the first k of each row on the device, download q, the scales
    and the status word."""
    m, ldx = xs.shape
    ldq = ldq or k
    dx = hip.Buffer.of(np.ascontiguousarray(xs))
    dq = hip.Buffer(max(m * ldq, 1))
    dq.zero()
    s_host = np.zeros(m, np.float32) if mode == L.SCALE_ROW_ABSMAX else np.ascontiguousarray(scale, np.float32)
    ds = hip.Buffer.of(s_host)
    dst = hip.Buffer.of(np.zeros(1, np.int32))
    say(f"quantize {L.TYPE_NAMES[x_type]}->{L.TYPE_NAMES[q_type]} mode={mode} m={m} k={k} ldx={ldx} ldq={ldq}")
    L.quantize(L.quantize_desc(x_type, q_type, m, k, dx.ptr, dq.ptr, ds.ptr, mode=mode, ldx=ldx, ldq=ldq,
                               status=dst.ptr))  # fmt: skip
    hip.synchronize()
    q = dq.download((m, ldq), np.uint8)[:, :k]
    s = ds.download((len(s_host),), np.float32)
    status = int(dst.download((1,), np.int32)[0])
    for b in (dx, dq, ds, dst):
        b.close()
    return q, s, status


def hard_rows(rng, m: int, ldx: int, q_type: int) -> tuple[np.ndarray, np.ndarray]:
    """m rows of ldx f32 values and a scale for each: normal rows at magnitudes from 1e-30 to 1e30, and rows built on
    the format's rounding boundaries at a power-of-two scale (so the boundaries are exact floats)."""
    x = rng.standard_normal((m, ldx)).astype(np.float32)
    x *= np.logspace(-30, 30, m, dtype=np.float64).astype(np.float32)[:, None]
    scale = np.logspace(-32, 28, m).astype(np.float32)
    if q_type == L.I8:
        grid = np.arange(-130, 131, dtype=np.float64) + 0.5
    else:
        v = np.array([H.oracle().oracle_decode(q_type, p) for p in range(128)])
        v = v[np.isfinite(v)]
        grid = np.concatenate([(v[1:] + v[:-1]) / 2, v])
        grid = np.concatenate([grid, -grid])
    for i in range(0, m, 3):  # ties and their neighbours, one ulp or two away
        s = np.float32(2.0 ** int(rng.integers(-20, 20)))
        t = (rng.choice(grid, ldx) * s).astype(np.float32)
        nudge = rng.integers(-2, 3, ldx).astype(np.int32)
        x[i] = (t.view(np.int32) + np.where(t != 0, nudge, 0)).view(np.float32)
        scale[i] = s
    if m > 1:
        x[1, : min(ldx, 8)] = np.array([0.0, -0.0, np.nan, 1e-45, -1e-40, 3e38, -3e38, 1.0], np.float32)[: min(ldx, 8)]
    if m > 2:
        scale[2] = np.float32(1e-41)  # below the shortcut's range: every element takes the exact path
    if m > 3:
        scale[3] = np.float32(-1.0)   # a scale the reference traps on (given modes)
    if m > 4:
        x[4, ldx // 2] = np.inf       # a computed scale the reference traps on
    return x, scale


SHAPES = [(1, 1, 1), (3, 7, 7), (17, 1000, 1000), (6, 1000, 1003), (5, 8200, 8200), (4, 9001, 9001), (64, 4096, 4096)]


@pytest.mark.parametrize("qname", list(Q_TYPES))
@pytest.mark.parametrize("xname", list(X_TYPES))
def test_every_type_and_mode_equals_the_oracle(xname, qname):
    x_type, q_type = X_TYPES[xname], Q_TYPES[qname]
    rng = np.random.default_rng(100 * x_type + q_type)
    for m, k, ldx in SHAPES:
        x, scale = hard_rows(rng, m, ldx, q_type)
        xs = patterns(x_type, x)
        for mname, mode in MODES.items():
            given = scale[:1] if mode == L.SCALE_TENSOR else scale
            want_q, want_s, want_status = H.quantize_rows(x_type, q_type, mode, xs, k, None if mode == 0 else given)
            got_q, got_s, got_status = run_quantize(x_type, q_type, mode, xs, k, None if mode == 0 else given)
            where = (xname, qname, mname, m, k, ldx)
            if mode == L.SCALE_ROW_ABSMAX:
                assert np.array_equal(got_s.view(np.uint32), want_s.view(np.uint32)), where
            bad = np.argwhere(got_q != want_q)
            assert bad.size == 0, (where, bad[:4].tolist(), [(int(got_q[tuple(b)]), int(want_q[tuple(b)])) for b in bad[:4]])
            assert got_status == want_status, (where, got_status, want_status)


def boundary_row(q_type: int, s: float, k: int) -> np.ndarray:
    """x for one row at scale s: every value of the 8-bit float's grid and every midpoint between neighbours, both
    signs, times s, and up to 3 f32 units either side of each; zeros after them to k elements."""
    codes = np.arange(128)
    v = np.array([H.oracle().oracle_decode(q_type, int(c)) for c in codes])
    v = v[np.isfinite(v)]
    grid = np.concatenate([v, (v[1:] + v[:-1]) / 2])
    grid = np.concatenate([grid, -grid])
    centre = (grid * s).astype(np.float32)
    xs = [(centre.view(np.int32) + np.where(centre != 0, np.int32(d), np.int32(0))).view(np.float32) for d in range(-3, 4)]
    x = np.concatenate(xs)
    assert len(x) <= k
    return np.concatenate([x, np.zeros(k - len(x), np.float32)])


@pytest.mark.parametrize("qname", ["e4m3", "e5m2"])
def test_the_hardware_conversion_decides_every_midpoint_as_the_oracle(qname):
    """The fast kernel converts the 8-bit floats with the hardware's conversion and settles elements near a midpoint
    of the grid from its neighbouring codes. Every grid value and midpoint, a few units either side, at scales whose
    reciprocal is inexact, given per row (the kernel's wave-a-row and workgroup-a-row forms), and bf16 rows whose
    computed scales make many quotients exact ties."""
    q_type = Q_TYPES[qname]
    scales = np.array([1.0, 3.0, 1 / 3, 0.37, 1.7e-6, 2.9e3, 0.1, 5.5e-3], np.float32)
    for k in (4096, 8200):
        x = np.stack([boundary_row(q_type, float(sc), k) for sc in scales])
        want_q, _, want_status = H.quantize_rows(L.F32, q_type, L.SCALE_ROW, x, k, scales)
        got_q, _, got_status = run_quantize(L.F32, q_type, L.SCALE_ROW, x, k, scales)
        bad = np.argwhere(got_q != want_q)
        assert bad.size == 0, (qname, k, bad[:4].tolist(), [(int(got_q[tuple(b)]), int(want_q[tuple(b)])) for b in bad[:4]])
        assert got_status == want_status
    # Computed scales: each row's largest magnitude a bf16 value with a short mantissa (1, 1.25, 1.5, 1.75, ...), so
    # that x / s is often exactly a midpoint.
    rng = np.random.default_rng(17 + q_type)
    m, k = 64, 4096
    x = rng.standard_normal((m, k)).astype(np.float32)
    tops = np.array([1.0, 1.25, 1.5, 1.75, 1.125, 1.375, 1.625, 1.875] * 8, np.float32) * np.float32(8.0)
    x = np.clip(x, -7.0, 7.0)
    x[np.arange(m), rng.integers(0, k, m)] = tops
    xs = patterns(L.BF16, x)
    want_q, want_s, _ = H.quantize_rows(L.BF16, q_type, L.SCALE_ROW_ABSMAX, xs, k)
    got_q, got_s, _ = run_quantize(L.BF16, q_type, L.SCALE_ROW_ABSMAX, xs, k)
    assert np.array_equal(got_s.view(np.uint32), want_s.view(np.uint32))
    bad = np.argwhere(got_q != want_q)
    assert bad.size == 0, (qname, bad[:4].tolist())


def test_a_padded_output_leaves_the_padding_alone():
    rng = np.random.default_rng(11)
    x = rng.standard_normal((8, 64)).astype(np.float32)
    got, _, _ = run_quantize(L.F32, L.I8, L.SCALE_ROW_ABSMAX, x, 48, ldq=72)
    want, _, _ = H.quantize_rows(L.F32, L.I8, L.SCALE_ROW_ABSMAX, x, 48)
    assert np.array_equal(got, want)


def test_w8a8_quantized_on_the_device_equals_the_oracle_chain():
    """Y = bf16((f32(Xq Wq^T) * sx[i]) * sw[j]) with Xq, Wq and their scales from the device quantize, W stored
    n x k (its output channels are its rows: the NT layout)."""
    rng = np.random.default_rng(8)
    m, n, k = 256, 512, 1024
    x = H.bf16_from_f32(rng.standard_normal((m, k)).astype(np.float32))
    w = H.bf16_from_f32((rng.standard_normal((n, k)) / 32).astype(np.float32))
    xq, sx, st1 = run_quantize(L.BF16, L.I8, L.SCALE_ROW_ABSMAX, x, k)
    wq, sw, st2 = run_quantize(L.BF16, L.I8, L.SCALE_ROW_ABSMAX, w, k)
    want_xq, want_sx, _ = H.quantize_rows(L.BF16, L.I8, 0, x, k)
    want_wq, want_sw, _ = H.quantize_rows(L.BF16, L.I8, 0, w, k)
    assert st1 == st2 == 0
    assert np.array_equal(xq, want_xq) and np.array_equal(wq, want_wq)
    assert np.array_equal(sx, want_sx) and np.array_equal(sw, want_sw)
    a, b = xq.view(np.int8), wq.view(np.int8)
    bufs = [hip.Buffer.of(np.ascontiguousarray(v)) for v in (a, b, sx, sw)]
    dc = hip.Buffer(m * n * 2)
    d = L.desc(L.I8, L.BF16, m, n, k, bufs[0].ptr, bufs[1].ptr, dc.ptr, trans_b=True, row_scale=bufs[2].ptr,
               col_scale=bufs[3].ptr)  # fmt: skip
    say("w8a8 gemm", L.select(d)["name"])
    L.run(d)
    hip.synchronize()
    got = dc.download((m, n), np.uint16)
    for buf in (*bufs, dc):
        buf.close()
    acc = H.gemm_i8(m, n, k, a, b, trans_b=True)
    assert np.array_equal(got, H.dequant(acc, sx, sw))
