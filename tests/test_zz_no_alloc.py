"""cairn_gemm_run_static, the entry point that allocates nothing: cairn_gemm_run with the split last round's workspace
taken from a scratch array the library holds on each GPU (CAIRN_GEMM_STATIC_SCRATCH bytes). Through the C ABI on the
GPU, against cairn_gemm_run given a workspace of its own of the same size, which plans the same split: the same bits,
on two calls in a row, the second smaller (the scratch keeps the first call's partial tiles, which the second must
not read). Both results also keep the multiply's contract against the exact product on sampled rows.
"""

from __future__ import annotations

import ctypes as C
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


def test_the_static_entry_equals_the_workspace_entry_on_two_calls_in_a_row():
    lib = L.load()
    rng = np.random.default_rng(707)
    ws = hip.Buffer(L.STATIC_SCRATCH)
    # 264 tiles (one round, then one tile an XCD over 32 stages), then 32 tiles (4 an XCD over 128 stages): the
    # selector splits both, within the scratch.
    for m, n, k in ((2048, 8448, 2048), (1024, 2048, 4096)):
        a = H.normal_bf16(rng, (m, k), 1.0)
        b = H.normal_bf16(rng, (k, n), 1.0)
        bias = H.normal_bf16(rng, (n,), 1.0)
        da, db, dbias = hip.Buffer.of(a), hip.Buffer.of(b), hip.Buffer.of(bias)
        dc_ref, dc_static = hip.Buffer(m * n * 2), hip.Buffer(m * n * 2)
        common = dict(bias=dbias.ptr, bias_type=L.BF16, act=L.ACT_GELU)
        ref = L.desc(L.BF16, L.BF16, m, n, k, da.ptr, db.ptr, dc_ref.ptr, workspace=ws.ptr,
                     workspace_bytes=L.STATIC_SCRATCH, **common)  # fmt: skip
        choice = L.select(ref)
        say(f"{m}x{n}x{k}: split {choice['split_tiles']} tiles over {choice['split_units']} units, "
            f"{choice['split_bytes'] >> 20} MiB of the {L.STATIC_SCRATCH >> 20} MiB scratch")  # fmt: skip
        assert choice["split_tiles"] > 0 and 0 < choice["split_bytes"] <= L.STATIC_SCRATCH
        L.run(ref)
        static = L.desc(L.BF16, L.BF16, m, n, k, da.ptr, db.ptr, dc_static.ptr, **common)
        assert lib.cairn_gemm_run_static(C.byref(static), None) == L.OK
        hip.synchronize()
        got_ref = dc_ref.download((m, n), np.uint16)
        got = dc_static.download((m, n), np.uint16)
        assert np.array_equal(got, got_ref), (m, n, k)
        rows = np.sort(rng.choice(m, 64, replace=False))
        exact, mag = H.exact_product(H.values(L.BF16, a[rows]), H.values(L.BF16, b))
        pre = exact + H.values(L.BF16, bias)[None, :]
        want = np.vectorize(H.oracle().oracle_gelu)(pre)
        room = 1.2 * H.bound(k, np.zeros(1), mag + np.abs(pre)) + 2.0**-8 * np.abs(want) * 1.01 + 1e-6
        assert H.outside(H.f32_from_bf16(got[rows]), want, room) == 0
        for x in (da, db, dbias, dc_ref, dc_static):
            x.close()
    ws.close()


def test_the_static_entry_refuses_a_workspace_and_a_split_past_its_scratch():
    lib = L.load()
    P = 1 << 20
    given = L.desc(L.BF16, L.BF16, 2048, 8448, 2048, P, P, P, workspace=P, workspace_bytes=1 << 30)
    assert lib.cairn_gemm_run_static(C.byref(given), None) == L.E_ARG
    # 256 units of the MLP forward's split need 128 MiB of partial tiles: more than the scratch holds.
    big = L.desc(L.BF16, L.BF16, 8192, 11008, 4096, P, P, P, split_units=256)
    status = lib.cairn_gemm_run_static(C.byref(big), None)
    assert status == L.E_SCRATCH, L.status_string(status)
    assert "scratch" in L.status_string(status)
