"""The split last round on the GPU (cairn_gemm_desc.workspace / split_units; cairn::tile::Split): where the output
tiles are not a whole number of rounds of the 256 CUs, the last round's tiles are shared along k by up to 256
workgroups, each writing partial tiles into the caller's workspace, and a fixup adds each tile's partials in k order
and applies the epilogue.

- The result keeps the multiply's contract against the exact fp64 product, through every epilogue and output type;
  int8 stays exact (an int32 sum in any order), so its int32 and dequantized outputs equal the unsplit kernel's.
- Its bits do not depend on timing: two runs give the same bits.
- Tiles outside the split round are the whole-tile pass's: bit for bit the unsplit result there.
- An explicit split (split_units > 0) that needs more workspace than given is refused, nothing queued.
"""

from __future__ import annotations

import sys

import numpy as np
import pytest

import helpers as H
from cairn_amd import hip
from cairn_amd import lib as L

pytestmark = pytest.mark.gpu


def say(*what):
    print("[gpu]", *what, flush=True)
    sys.stdout.flush()


def gemm(ab, out, m, n, k, a, b, *, split: bool, units: int = 0, c_init=None, **kw):
    """One cairn_gemm_run on the null stream: with the workspace cairn_gemm_workspace asks for (split) or with none;
    returns (c, the selector's choice)."""
    dtype = {L.F32: np.float32, L.BF16: np.uint16, L.F16: np.uint16, L.I32: np.int32}[out]
    host = np.zeros((m, n), dtype) if c_init is None else np.ascontiguousarray(c_init, dtype=dtype)
    extra = {name: hip.Buffer.of(np.ascontiguousarray(v)) for name, v in kw.items() if isinstance(v, np.ndarray)}
    args = {name: (extra[name].ptr if name in extra else v) for name, v in kw.items()}
    da, db, dc = hip.Buffer.of(np.ascontiguousarray(a)), hip.Buffer.of(np.ascontiguousarray(b)), hip.Buffer.of(host)
    probe = L.desc(ab, out, m, n, k, da.ptr, db.ptr, dc.ptr, split_units=units if split else -1, **args)
    bytes_ = L.workspace(probe) if split else 0
    ws = hip.Buffer(max(bytes_, 256)) if split else None
    d = L.desc(ab, out, m, n, k, da.ptr, db.ptr, dc.ptr, workspace=ws.ptr if ws else None, workspace_bytes=bytes_,
               split_units=units if split else -1, **args)  # fmt: skip
    choice = L.select(d)
    say(f"{L.TYPE_NAMES[ab]}->{L.TYPE_NAMES[out]} {m}x{n}x{k} on {choice['name']}: split {choice['split_tiles']} tiles "
        f"over {choice['split_units']} units, {bytes_ >> 20} MiB")  # fmt: skip
    L.run(d)
    hip.synchronize()
    got = dc.download(host.shape, dtype)
    for x in (da, db, dc, ws, *extra.values()):
        if x is not None:
            x.close()
    return got, choice


def split_mask(m, n, split_tiles, tile=256, group=4, cus=256):
    """Which outputs the split tiles cover: the ids the planner splits (the last ids of each XCD's block of the
    xcd_order, 8 blocks where the tile count divides into them), mapped to tiles as cairn::tile::tile_at does
    (`group` tile rows walked together)."""
    tm_count, tn_count = (m + tile - 1) // tile, (n + tile - 1) // tile
    total = tm_count * tn_count
    xcds = 8 if total % 8 == 0 else 1
    block = total // xcds
    per = cus // xcds
    first = block // per * per
    ids = [x * block + i for x in range(xcds) for i in range(first, block)]
    assert len(ids) == split_tiles
    mask = np.zeros((m, n), dtype=bool)
    for i in ids:
        per_group = group * tn_count
        top = (i // per_group) * group
        rows = min(tm_count - top, group)
        local = i - (i // per_group) * per_group
        r, c = top + local % rows, local // rows
        mask[r * tile : (r + 1) * tile, c * tile : (c + 1) * tile] = True
    return mask


LAYOUTS = [(False, False), (False, True), (True, False), (True, True)]


@pytest.mark.parametrize("trans_a,trans_b", LAYOUTS)
def test_a_split_round_keeps_the_contract_and_its_bits_on_every_layout(trans_a, trans_b):
    """264 tiles (one round and 8 tiles) with random bf16 operands, bias and GELU into bf16: within the contract
    (through GELU's slope) of the exact product, the same bits twice, and outside the split tiles the unsplit bits."""
    rng = np.random.default_rng(17 + 2 * trans_a + trans_b)
    m, n, k = 2048, 8448, 1024
    a = H.normal_bf16(rng, (k, m) if trans_a else (m, k), 1.0)
    b = H.normal_bf16(rng, (n, k) if trans_b else (k, n), 1.0)
    bias = H.normal_bf16(rng, (n,), 1.0)
    kw = dict(trans_a=trans_a, trans_b=trans_b, bias=bias, bias_type=L.BF16, act=L.ACT_GELU)
    got, ch = gemm(L.BF16, L.BF16, m, n, k, a, b, split=True, **kw)
    assert ch["split_tiles"] == 8 and ch["split_units"] > 1
    again, _ = gemm(L.BF16, L.BF16, m, n, k, a, b, split=True, **kw)
    assert np.array_equal(got, again), "the split round's bits depend on timing"
    whole, ch0 = gemm(L.BF16, L.BF16, m, n, k, a, b, split=False, **kw)
    assert ch0["split_tiles"] == 0
    mask = split_mask(m, n, 8)
    say(f"outputs that differ from the unsplit run: {int((got != whole).sum())}, in the split tiles {int(mask.sum())}")
    assert np.array_equal(got[~mask], whole[~mask]), "a tile of the whole-tile pass changed"
    rows = np.concatenate([np.arange(0, 64), np.nonzero(mask.any(axis=1))[0]])
    A = H.values(L.BF16, a.T if trans_a else a)[rows]
    B = H.values(L.BF16, b.T if trans_b else b)
    exact, mag = H.exact_product(A, B)
    pre = exact + H.values(L.BF16, bias)[None, :]
    want = np.vectorize(H.oracle().oracle_gelu)(pre)
    room = 1.2 * H.bound(k, np.zeros(1), mag + np.abs(pre)) + 2.0**-8 * np.abs(want) * 1.01 + 1e-6
    assert H.outside(H.f32_from_bf16(got[rows]), want, room) == 0


def test_int8_through_a_split_round_is_exact():
    """int32 sums are exact in any order: the split result equals the unsplit one, as int32 and through the dequant
    epilogue into bf16 (bit for bit the oracle's order)."""
    rng = np.random.default_rng(88)
    m, n, k = 2048, 8448, 2048
    a = rng.integers(-127, 128, (m, k), dtype=np.int8)
    b = rng.integers(-127, 128, (k, n), dtype=np.int8)
    got, ch = gemm(L.I8, L.I32, m, n, k, a, b, split=True)
    assert ch["split_tiles"] == 8
    rows = np.nonzero(split_mask(m, n, 8).any(axis=1))[0][::4]
    assert np.array_equal(got[rows].astype(np.float64), a[rows].astype(np.float64) @ b.astype(np.float64))
    sa = rng.uniform(1e-3, 1e-2, m).astype(np.float32)
    sb = rng.uniform(1e-3, 1e-2, n).astype(np.float32)
    deq, _ = gemm(L.I8, L.BF16, m, n, k, a, b, split=True, row_scale=sa, col_scale=sb)
    assert np.array_equal(deq[rows], H.dequant(got[rows], sa[rows], sb))


def test_a_split_round_accumulates_into_f32_c():
    """c += a b with f32 c: the fixup adds the old value last, as the whole-tile epilogue does; exact data, so every
    output is exact."""
    m, n, k = 2048, 8448, 512
    a = H.encode(L.BF16, H.tile_values(m * k, 61)).reshape(m, k)
    b = H.encode(L.BF16, H.tile_values(k * n, 62)).reshape(k, n)
    c0 = (H.tile_values(m * n, 63) / 8).astype(np.float32).reshape(m, n)
    got, ch = gemm(L.BF16, L.F32, m, n, k, a, b, split=True, units=64, c_init=c0, accumulate=True)
    assert ch["split_units"] == 64
    rows = np.nonzero(split_mask(m, n, 8).any(axis=1))[0][::8]
    exact, _ = H.gemm_f64(L.BF16, len(rows), n, k, np.ascontiguousarray(a[rows]), b)
    assert np.array_equal(got[rows].astype(np.float64), c0[rows].astype(np.float64) + exact)


@pytest.mark.parametrize("fmt", [L.F8E4M3, L.F16])
def test_the_other_operand_types_split_too(fmt):
    rng = np.random.default_rng(90 + fmt)
    m, n, k = 2048, 8448, 1024

    def operand(shape):
        if fmt == L.F16:
            return rng.standard_normal(shape).astype(np.float16).view(np.uint16)
        p = rng.integers(0, 256, shape, dtype=np.uint8)  # every finite E4M3 pattern at random
        bad = ~np.isfinite(H.values(fmt, p))
        p[bad] &= 0xBF
        return p

    a, b = operand((m, k)), operand((k, n))
    # The selector widens the 8-bit floats into the 128 x 128 kernel, which never splits: the ring's kernel on the fp8
    # matrix core is named (at this k its grouped adds stay within the contract).
    kernel = {"kernel": L.kernel_named("cairn_wave_f8e4m3_nn_256x256")} if fmt == L.F8E4M3 else {}
    got, ch = gemm(fmt, L.F32, m, n, k, a, b, split=True, **kernel)
    assert ch["split_tiles"] == 8
    rows = np.nonzero(split_mask(m, n, 8).any(axis=1))[0][::4]
    exact, mag = H.exact_product(H.values(fmt, a[rows]), H.values(fmt, b))
    assert H.outside(got[rows], exact, H.bound(k, np.zeros(1), mag)) == 0


def test_the_mlp_forward_splits_its_last_round_deterministically():
    """C3's forward (8192 x 11008 x 4096, bias + GELU, bf16 out) with its split asked for: 1376 tiles, 5 whole rounds
    and 96 tiles shared by 256 units. Two runs, the same bits; 256 sampled rows of the split round against the exact
    product."""
    rng = np.random.default_rng(3)
    m, k, n = 8192, 4096, 11008
    x = H.normal_bf16(rng, (m, k), 1.0)
    w = H.normal_bf16(rng, (k, n), 0.02)
    bias = H.normal_bf16(rng, (n,), 0.02)
    kw = dict(bias=bias, bias_type=L.BF16, act=L.ACT_GELU)
    y, ch = gemm(L.BF16, L.BF16, m, n, k, x, w, split=True, units=256, **kw)  # asked for: the selector would not
    assert ch["split_tiles"] == 96 and ch["efficiency"] >= 0.97
    y2, _ = gemm(L.BF16, L.BF16, m, n, k, x, w, split=True, units=256, **kw)
    assert np.array_equal(y, y2)
    rows = np.sort(rng.choice(np.nonzero(split_mask(m, n, 96).any(axis=1))[0], 256, replace=False))
    exact, mag = H.exact_product(H.values(L.BF16, x[rows]), H.values(L.BF16, w))
    pre = exact + H.values(L.BF16, bias)[None, :]
    want = np.vectorize(H.oracle().oracle_gelu)(pre)
    room = 1.2 * H.bound(k, np.zeros(1), mag + np.abs(pre)) + 2.0**-8 * np.abs(want) * 1.01 + 1e-6
    assert H.outside(H.f32_from_bf16(y[rows]), want, room) == 0


def test_an_explicit_split_larger_than_its_workspace_is_refused():
    P = 1 << 20
    d = L.desc(L.BF16, L.BF16, 2048, 8448, 1024, P, P, P, workspace=P, workspace_bytes=1 << 20, split_units=200)
    s = L.load().cairn_gemm_run(d, None)
    assert s == L.E_SCRATCH, L.status_string(s)
