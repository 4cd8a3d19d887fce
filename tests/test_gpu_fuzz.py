"""Seeded random problems through cairn_gemm_run on the GPU, each against the exact product on sampled rows: every
operand type, layout, output type and epilogue, extents with tails in every direction, padded leading dimensions, and a
workspace for the split last round where the draw gives one. The selector picks the kernel, so the draws reach the ring,
MFMA, generic and skinny families (and the split where a problem's last round qualifies); each case prints itself
before it runs.

The checks are the multiply's contract (tests/soundness/test_tensor.py's bound, (k + 1) 2^-22 (|c| + sum |a b|)),
carried through the epilogue's steps: the scales multiply the bound, GELU's slope (at most 1.13) stretches it, each f32
step adds its rounding, and the output type its own (bf16 2^-8, f16 2^-11 relative). int8 into int32 is exact; int8
into bf16 with scales alone is the oracle's dequant, bit for bit."""

from __future__ import annotations

import math
import sys

import numpy as np
import pytest
from scipy.special import erfc

import helpers as H
from cairn_amd import hip
from cairn_amd import lib as L

pytestmark = pytest.mark.gpu

# Three draws in four from extents the tiled kernels' 16-byte chunks fit (multiples of 16, at least a 256-wide
# tile), with tails against 256; the rest from any extents (tails in every direction, the generic kernel's).
TILED = [256, 272, 512, 528, 640, 1024, 1040, 1536, 2048]
DEPTHS_TILED = [16, 64, 128, 272, 528, 1024, 2048, 4096]
SIZES = [1, 2, 3, 7, 16, 33, 100, 257, 512, 640, 1000, 1024, 1536]
DEPTHS = [8, 16, 24, 40, 64, 72, 128, 200, 264, 520, 1000, 1024, 2048, 4104]
CASES = 72


def say(*what):
    print("[gpu]", *what, flush=True)
    sys.stdout.flush()


def operand(ab: int, shape, rng) -> np.ndarray:
    if ab == L.I8:
        return rng.integers(-127, 128, shape, dtype=np.int8)
    if ab == L.BF16:
        return H.normal_bf16(rng, shape, 1.0)
    if ab == L.F16:
        return rng.standard_normal(shape).astype(np.float16).view(np.uint16)
    p = rng.integers(0, 256, shape, dtype=np.uint8)  # every finite pattern of the 8-bit float at random
    p[~np.isfinite(H.values(ab, p))] &= 0xBF
    return p


def padded(rows: int, cols: int, pad: int, x: np.ndarray) -> np.ndarray:
    """x (rows x cols) stored with leading dimension cols + pad."""
    out = np.zeros((rows, cols + pad), dtype=x.dtype)
    out[:, :cols] = x
    return out


def draw(rng, case: int) -> dict:
    ab = int(rng.choice([L.BF16, L.BF16, L.F16, L.I8, L.F8E4M3, L.F8E5M2]))
    ta, tb = bool(rng.integers(2)), bool(rng.integers(2))
    if ab == L.BF16 and case % 4 == 0:  # decode-shaped: the skinny family
        ta, tb = False, True
        m = int(rng.choice([1, 2, 3, 4, 5, 8, 16]))
    elif rng.random() < 0.75:
        m = int(rng.choice(TILED))
    else:
        m = int(rng.choice(SIZES))
    if rng.random() < 0.75:
        n, k = int(rng.choice(TILED)), int(rng.choice(DEPTHS_TILED))
    else:
        n, k = int(rng.choice(SIZES)), int(rng.choice(DEPTHS))
    while m * n * k > 1_500_000_000:
        k = max(8, k // 2)
    if ab == L.I8:
        out = int(rng.choice([L.I32, L.BF16]))
    elif ab in (L.F8E4M3, L.F8E5M2):
        out = int(rng.choice([L.F32, L.BF16]))
    else:
        out = int(rng.choice([L.F32, L.BF16, L.F16]))
    epi = {}
    if out != L.I32:
        if rng.random() < 0.4:
            epi["scales"] = True
        if rng.random() < 0.4:
            epi["bias"] = int(rng.choice([L.F32, L.BF16]))
        epi["act"] = int(rng.choice([L.ACT_NONE, L.ACT_NONE, L.ACT_RELU, L.ACT_GELU]))
        if out == L.F32 and rng.random() < 0.3 and not epi.get("scales"):
            epi["accumulate"] = True
    if ab in (L.F8E4M3, L.F8E5M2) or out == L.F16:
        epi.pop("scales", None)  # keep the 8-bit floats' large products and f16's range apart from the scales
    pads = [int(rng.choice([0, 0, 0, 16, 32])) for _ in range(3)]
    split = rng.random() < 0.35
    return {"ab": ab, "out": out, "m": m, "n": n, "k": k, "ta": ta, "tb": tb, "epi": epi, "pads": pads, "split": split}


def test_random_problems_keep_the_contract():
    rng = np.random.default_rng(20261202)
    for case in range(CASES):
        p = draw(rng, case)
        ab, out, m, n, k, ta, tb, epi = p["ab"], p["out"], p["m"], p["n"], p["k"], p["ta"], p["tb"], p["epi"]
        pa, pb, pc = p["pads"]
        say(f"case {case}: {L.TYPE_NAMES[ab]}->{L.TYPE_NAMES[out]} {m}x{n}x{k} ta={ta} tb={tb} pads={p['pads']} "
            f"epi={epi} split={p['split']}")  # fmt: skip
        a = operand(ab, (k, m) if ta else (m, k), rng)
        b = operand(ab, (n, k) if tb else (k, n), rng)
        a_st, b_st = padded(*a.shape, pa, a), padded(*b.shape, pb, b)
        odt = {L.F32: np.float32, L.BF16: np.uint16, L.F16: np.uint16, L.I32: np.int32}[out]
        c0 = rng.uniform(-4, 4, (m, n)).astype(np.float32) if epi.get("accumulate") else np.zeros((m, n), np.float32)
        c_st = padded(m, n, pc, c0.astype(odt) if out != L.F32 else c0)
        rs = rng.uniform(0.25, 2.0, m).astype(np.float32) if epi.get("scales") else None
        cs = rng.uniform(0.25, 2.0, n).astype(np.float32) if epi.get("scales") else None
        bias_t = epi.get("bias")
        bias = None
        if bias_t == L.F32:
            bias = rng.uniform(-8, 8, n).astype(np.float32)
        elif bias_t == L.BF16:
            bias = H.bf16_from_f32(rng.uniform(-8, 8, n).astype(np.float32))
        bufs = {name: hip.Buffer.of(np.ascontiguousarray(x)) for name, x in
                (("a", a_st), ("b", b_st), ("c", c_st), ("rs", rs), ("cs", cs), ("bias", bias)) if x is not None}  # fmt: skip
        kw = dict(trans_a=ta, trans_b=tb, lda=a_st.shape[1], ldb=b_st.shape[1], ldc=c_st.shape[1],
                  accumulate=bool(epi.get("accumulate")), act=epi.get("act", L.ACT_NONE),
                  bias=bufs["bias"].ptr if "bias" in bufs else None, bias_type=bias_t or L.F32,
                  row_scale=bufs["rs"].ptr if "rs" in bufs else None, col_scale=bufs["cs"].ptr if "cs" in bufs else None)  # fmt: skip
        d = L.desc(ab, out, m, n, k, bufs["a"].ptr, bufs["b"].ptr, bufs["c"].ptr, **kw)
        if p["split"]:
            need = L.workspace(d)
            bufs["ws"] = hip.Buffer(max(need, 256))
            d = L.desc(ab, out, m, n, k, bufs["a"].ptr, bufs["b"].ptr, bufs["c"].ptr, workspace=bufs["ws"].ptr,
                       workspace_bytes=need, **kw)  # fmt: skip
        choice = L.select(d)
        say(f"    -> {choice['name']} split {choice['split_tiles']} tiles over {choice['split_units']} units")
        L.run(d)
        hip.synchronize()
        got_st = bufs["c"].download(c_st.shape, odt)
        for x in bufs.values():
            x.close()
        got = got_st[:, :n]
        rows = np.unique(np.concatenate([rng.choice(m, min(m, 40), replace=False), [m - 1]]))
        A = a.T if ta else a
        B = b.T if tb else b
        if ab == L.I8:
            acc = A[rows].astype(np.int64) @ B.astype(np.int64)
            if out == L.I32:
                assert np.array_equal(got[rows], acc.astype(np.int32)), case
                continue
            if not epi.get("bias") and epi.get("act", 0) == L.ACT_NONE and rs is not None:
                want = H.dequant(acc.astype(np.int32), rs[rows], cs)
                assert np.array_equal(got[rows], want), case
                continue
            exact, mag = acc.astype(np.float64), np.abs(A[rows].astype(np.float64)) @ np.abs(B.astype(np.float64))
            acc_room = np.abs(exact) * 2.0**-24  # the exact int32 sum converted to f32
        else:
            exact, mag = H.exact_product(H.values(ab, A[rows]), H.values(ab, B))
            acc_room = H.bound(k, np.zeros(1), mag)
        s = (rs[rows][:, None].astype(np.float64) if rs is not None else 1.0) * (cs[None, :].astype(np.float64) if cs is not None else 1.0)
        pre = exact * s
        if bias is not None:
            pre = pre + H.values(L.BF16, bias)[None, :] if bias_t == L.BF16 else pre + bias.astype(np.float64)[None, :]
        act = epi.get("act", L.ACT_NONE)
        if act == L.ACT_RELU:
            want = np.maximum(pre, 0.0)
        elif act == L.ACT_GELU:
            want = 0.5 * pre * erfc(-pre / math.sqrt(2.0))  # no cancellation, unlike 1 + erf
        else:
            want = pre
        room = (1.2 if act == L.ACT_GELU else 1.0) * (acc_room * np.abs(s) + 4 * 2.0**-24 * (np.abs(pre) + np.abs(exact * s)))
        room = room + (1e-5 * np.abs(want) if act == L.ACT_GELU else 0.0) + 1e-30  # GELU's own error: 7.7e-6 at most
        if epi.get("accumulate"):
            want = want + c0[rows].astype(np.float64)
            room = room + H.bound(k, c0[rows], np.zeros(1)) + 2.0**-24 * np.abs(want)
        if out == L.BF16:
            v = H.f32_from_bf16(got[rows])
            room = room + 2.0**-8 * np.abs(want) * 1.01
        elif out == L.F16:
            v = H.f32_from_f16(got[rows])
            room = room + 2.0**-11 * np.abs(want) * 1.01 + 2.0**-25
        else:
            v = got[rows]
        bad = H.outside(v, want, room)
        assert bad == 0, (case, p, bad)
    say(f"{CASES} random problems within the contract")
