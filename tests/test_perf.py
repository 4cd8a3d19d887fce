"""The multiply's pricing (cairn_amd/perf.py) on the CPU: the MI355X card keeps CAIRN's card schema, the roofline is the
reference's formula, and the prediction prices the kernel the selector will launch with that kernel's measured rate."""

from __future__ import annotations

import math

import pytest

from cairn_amd import lib as L
from cairn_amd import perf

P = 1 << 20  # an aligned stand-in address: the selector reads alignment only
# The fields of the reference's Device (src/cairn/perf/profile.py:75-112), without defaults first: the card's device
# block may hold these names only, and must hold the first nine, or Profile.load cannot build it.
REQUIRED = ["name", "sms", "cores_per_sm", "ghz", "dram_gbps", "flops", "launch_ns", "link_gbps", "link_ns"]
OPTIONAL = ["memory_efficiency", "occupancy_to_saturate", "registers_per_sm", "registers_per_block",
            "registers_per_thread", "threads_per_sm", "threads_per_block", "blocks_per_sm", "shared_per_sm",
            "shared_per_block", "warp", "partitions", "register_unit", "shared_unit", "shared_reserved",
            "shared_bytes_per_clock", "memory_latency_ns", "compute_capability", "target"]  # fmt: skip


def test_the_card_keeps_the_reference_schema():
    data = perf.card()
    assert data["schema"] == "cairn.machine/1" and data["origin"] in ("measured", "specification")
    assert data["host"] is None  # a device card: a device and no host (profile.py:194-199)
    device = data["device"]
    assert set(REQUIRED) <= set(device) <= set(REQUIRED + OPTIONAL), set(device) ^ set(REQUIRED + OPTIONAL)
    assert device["flops"]["tensor_f16"] == pytest.approx(256 * 4096 * 2.4, rel=1e-4)  # ops per ns
    assert device["flops"]["tensor_i8"] == 2 * device["flops"]["tensor_bf16"]
    assert device["warp"] == 64 and device["shared_per_block"] == 160 * 1024
    assert set(data["source"]["assumed"]) | set(data["source"]["published"]) <= set(REQUIRED + OPTIONAL)


def test_every_kernel_of_the_library_has_a_measured_rate():
    g = perf.card()["gemm"]
    assert g["origin"] == "measured"
    for k in L.kernels():
        if k["family"] == "skinny":
            continue
        entry = g["kernels"][k["name"]]
        assert entry["family"] == k["family"] and 0.0 < entry["frac"] < 1.0, k["name"]
    assert set(g["skinny"]) == {"m1", "m4", "m16"} and all(0.0 < v < 1.0 for v in g["skinny"].values())


def test_the_roofline_is_the_reference_formula():
    d = perf.card()["device"]
    n = 4096
    r = perf.tensor(n, n, n, L.BF16)
    moved = 2 * n * n * 2 + 2 * n * n * 4  # a and b bf16 once; c f32 read and written (work.py:466-471)
    assert r["memory_ns"] == pytest.approx(moved / (8000.0 * 0.85))
    assert r["compute_ns"] == pytest.approx(2.0 * n**3 / d["flops"]["tensor_f16"])
    assert r["ns"] == pytest.approx(d["launch_ns"] + r["compute_ns"]) and r["bound"] == "tensor cores"
    skinny = perf.tensor(1, 14336, 4096, L.BF16)
    assert skinny["bound"] == "device memory"
    assert perf.tensor(8, 8, 8, L.F8E4M3)["bound"] == "launch"
    # Every format at the f16 rate in the reference's model: an 8-bit float costs the same operations.
    assert perf.tensor(n, n, n, L.F8E4M3)["compute_ns"] == r["compute_ns"]


def test_the_prediction_prices_the_kernel_the_selector_launches():
    data = perf.card()
    d, g = data["device"], data["gemm"]
    n = 4096
    desc = L.desc(L.BF16, L.BF16, n, n, n, P, P, P)
    p = perf.predict(desc, data)
    assert p["kernel"] == L.select(desc)["name"] == "cairn_wave_bf16_nn_256x256"
    rate = g["kernels"][p["kernel"]]["frac"]
    assert p["ns"] == pytest.approx(d["launch_ns"] + 2.0 * n**3 / (d["flops"]["tensor_bf16"] * rate))
    # A tiling that leaves CUs idle costs more than its operations alone: 520 x 4096 is 3 x 16 tiles on 256 CUs.
    ragged = perf.predict(L.desc(L.BF16, L.BF16, 520, n, n, P, P, P), data)
    assert ragged["tiling_efficiency"] < 0.2 and ragged["compute_ns"] > 4.0 * 2.0 * 520 * n * n / (
        d["flops"]["tensor_bf16"] * rate)
    # fp8 as the selector runs it (widened to f16) at the f16 peak; on the fp8 matrix core (named) at the fp8 peak.
    f8 = perf.predict(L.desc(L.F8E4M3, L.BF16, n, n, n, P, P, P), data)
    assert f8["kernel"].startswith("cairn_mfma_f8e4m3") and math.isclose(
        f8["compute_ns"], 2.0 * n**3 / (d["flops"]["tensor_f16"] * g["kernels"][f8["kernel"]]["frac"]), rel_tol=1e-9)
    core = L.desc(L.F8E4M3, L.BF16, n, n, n, P, P, P, kernel=L.kernel_named("cairn_wave_f8e4m3_nn_256x256"))
    f8c = perf.predict(core, data)
    assert f8c["kernel"] == "cairn_wave_f8e4m3_nn_256x256" and math.isclose(
        f8c["compute_ns"], 2.0 * n**3 / (d["flops"]["tensor_f8"] * g["kernels"][f8c["kernel"]]["frac"]), rel_tol=1e-9)
    # The decode shape: the skinny kernel at its measured share of HBM.
    dec = perf.predict(L.desc(L.BF16, L.BF16, 1, 14336, 4096, P, P, P, trans_b=True), data)
    moved = (4096 + 14336 * 4096) * 2 + 14336 * 2
    assert dec["kernel"] == "cairn_skinny_bf16_nt" and dec["bound"] == "device memory"
    assert dec["ns"] == pytest.approx(d["launch_ns"] + moved / (8000.0 * g["skinny"]["m1"]))


def test_the_card_is_rewritten_from_a_calibration_run():
    data = perf.card()
    run = {"calibration": {"cairn_x": {"family": "wave", "problem": "4096^3", "tflops": 1000.0, "frac": 0.4}},
           "skinny": {"m1": {"frac": 0.6}, "m4": {"frac": 0.55}, "m16": {"frac": 0.5}}}  # fmt: skip
    new = perf.card_from(run, data)
    assert new["gemm"]["kernels"] == {"cairn_x": {"family": "wave", "problem": "4096^3", "tflops": 1000.0, "frac": 0.4}}
    assert new["gemm"]["skinny"] == {"m1": 0.6, "m4": 0.55, "m16": 0.5} and new["device"] == data["device"]
