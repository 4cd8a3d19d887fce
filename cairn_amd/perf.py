"""The multiply's pricing for the perf model: an MI355X machine card in CAIRN's card schema, the reference's roofline
for a tensor-core multiply, and a prediction that knows which kernel `cairn_gemm_run` will launch.

- The card (cards/mi355x.json) is a `cairn.machine/1` profile, the schema of src/cairn/perf/profile.py:164-184. Its
  `device` block has exactly the fields of the reference's Device (profile.py:75-112), from AMD's published figures.
  A top-level `gemm` block, which the reference's loader keeps in Profile.source, holds what this library measured:
  each kernel's rate on a problem its tiles cover whole (`python3 bench.py --only calibrate`), and the skinny
  kernel's share of HBM bandwidth.
- `tensor` restates the reference's price of a device multiply (src/cairn/perf/model.py:139-153; the work it prices,
  src/cairn/perf/work.py:459-480): a launch, then the larger of the bytes at the sustained bandwidth and the
  operations at the tensor peak.
- `predict` prices what launch will run: the selector's kernel (cairn_gemm_select, no GPU), the share of the machine
  its tiling keeps busy, and that kernel's measured rate.

Usage: `python3 -m cairn_amd.perf --card-from calibration.json` writes the card's gemm block from a calibration run's
JSON line; `python3 -m cairn_amd.perf M N K [type]` prints both prices.
"""

from __future__ import annotations

import argparse
import json
import sys
from pathlib import Path

from . import lib as L

CARD = Path(__file__).resolve().parent / "cards" / "mi355x.json"
SIZE = {L.F32: 4, L.F16: 2, L.BF16: 2, L.F8E4M3: 1, L.F8E5M2: 1, L.I8: 1, L.I32: 4}
PEAK_KEY = {L.F16: "tensor_f16", L.BF16: "tensor_bf16", L.F8E4M3: "tensor_f8", L.F8E5M2: "tensor_f8",
            L.I8: "tensor_i8"}  # fmt: skip


def card(path: Path = CARD) -> dict:
    """The card as data (the reference's Profile.load reads the same file: its `device` block is a Device)."""
    data = json.loads(Path(path).read_text(encoding="utf-8"))
    if data.get("schema") != "cairn.machine/1":
        raise ValueError(f"{path} is not a cairn.machine/1 profile")
    return data


def tensor(m: int, n: int, k: int, ab_type: int, data: dict | None = None) -> dict:
    """The reference's price of mma_unordered on the device (model.py:139-153): bytes a m x k + b k x n of the storage
    float read once, c m x n f32 read and written once (work.py:466-471); 2mnk operations at the tensor peak, every
    format at the f16 rate as the reference widens 8-bit floats; time = launch + max(memory, compute) in ns."""
    d = (data or card())["device"]
    size = SIZE[ab_type]
    moved = m * k * size + k * n * size + 2.0 * m * n * 4.0
    work = 2.0 * m * n * k
    peak = d["flops"].get("tensor_f16", d["flops"]["f32"])
    memory = moved / (d["dram_gbps"] * d["memory_efficiency"])
    compute = work / peak
    bound = "launch" if d["launch_ns"] > max(memory, compute) else "device memory" if memory >= compute else "tensor cores"
    return {"ns": d["launch_ns"] + max(memory, compute), "bound": bound, "memory_ns": memory, "compute_ns": compute,
            "launch_ns": d["launch_ns"], "peak_ops_per_ns": peak}  # fmt: skip


def predict(desc: L.Desc, data: dict | None = None) -> dict:
    """What cairn_gemm_run(desc) takes: the selector's kernel at its measured rate, on the share of the machine its
    tiling keeps busy (workgroups over CU slots, edge tiles); the skinny kernel at its measured share of HBM. Every
    input is known before a launch: no GPU is touched."""
    data = data or card()
    d, g = data["device"], data["gemm"]
    choice = L.select(desc)
    m, n, k = int(desc.m), int(desc.n), int(desc.k)
    a_size, c_size = SIZE[desc.ab_type], SIZE[desc.c_type]
    moved = (m * k + k * n) * a_size + m * n * c_size * (2 if desc.accumulate else 1)
    work = 2.0 * m * n * k
    if choice["family"] == "skinny":
        share = g["skinny"][f"m{1 if m <= 1 else 4 if m <= 4 else 16}"]
        memory = moved / (d["dram_gbps"] * share)
        return {"ns": d["launch_ns"] + memory, "kernel": choice["name"], "bound": "device memory",
                "memory_ns": memory, "hbm_share": share}  # fmt: skip
    rate = g["kernels"][choice["name"]]["frac"]
    # The MFMA family widens the 8-bit floats to f16: its rates are shares of the f16 peak.
    widened = choice["family"] == "mfma" and desc.ab_type in (L.F8E4M3, L.F8E5M2)
    peak = d["flops"]["tensor_f16" if widened else PEAK_KEY[desc.ab_type]] * rate * choice["efficiency"]
    compute = work / peak
    memory = moved / (d["dram_gbps"] * d["memory_efficiency"])
    return {"ns": d["launch_ns"] + max(memory, compute), "kernel": choice["name"],
            "bound": "device memory" if memory > compute else "tensor cores", "compute_ns": compute,
            "memory_ns": memory, "kernel_rate": rate, "tiling_efficiency": choice["efficiency"]}  # fmt: skip


def card_from(calibration: dict, data: dict | None = None) -> dict:
    """The card with its gemm block replaced by a calibration run's figures (bench.py --only calibrate)."""
    data = json.loads(json.dumps(data or card()))
    data["gemm"]["kernels"] = {name: {"family": v["family"], "problem": v["problem"], "tflops": v["tflops"],
                                      "frac": v["frac"]} for name, v in calibration["calibration"].items()}  # fmt: skip
    data["gemm"]["skinny"] = {m: round(v["frac"], 4) for m, v in calibration["skinny"].items()}
    return data


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser(prog="python3 -m cairn_amd.perf")
    ap.add_argument("--card-from", type=Path, help="a calibration run's JSON line: rewrite the card's gemm block")
    ap.add_argument("shape", nargs="*", type=int, help="M N K")
    ap.add_argument("--type", default="bf16", choices=list(L.TYPE_NAMES.values()))
    ap.add_argument("--trans-a", action="store_true")
    ap.add_argument("--trans-b", action="store_true", help="b stored n x k (the decode layout)")
    args = ap.parse_args(argv)
    if args.card_from:
        line = next(x for x in args.card_from.read_text().splitlines() if x.startswith("{"))
        CARD.write_text(json.dumps(card_from(json.loads(line)), indent=1) + "\n", encoding="utf-8")
        print(f"wrote {CARD}")
        return 0
    if len(args.shape) != 3:
        ap.error("give M N K")
    m, n, k = args.shape
    t = {v: key for key, v in L.TYPE_NAMES.items()}[args.type]
    out = L.I32 if t == L.I8 else L.BF16
    p = 1 << 20  # an aligned stand-in address: the selector reads alignment only
    d = L.desc(t, out, m, n, k, p, p, p, trans_a=args.trans_a, trans_b=args.trans_b)
    print(json.dumps({"roofline": tensor(m, n, k, t), "predicted": predict(d)}))
    return 0


if __name__ == "__main__":
    sys.exit(main())
