"""bench.py's reading of rocprofv3 output on the CPU: the kernel-trace table's averages (all launches, and the last K,
a bench section's timed launches after its warm-up) and the `traffic:` line the JSON record's roofline takes from
the committed counter summary. Synthetic CSV files of rocprofv3's layout; no GPU."""

from __future__ import annotations

import csv
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402

FIELDS = ["Kernel_Name", "Grid_Size_X", "Grid_Size_Y", "Grid_Size_Z", "Start_Timestamp", "End_Timestamp"]


def write_trace(path: Path, rows: list[tuple[str, int, int, int]]) -> None:
    with path.open("w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=FIELDS)
        w.writeheader()
        for name, grid, start, ns in rows:
            w.writerow({"Kernel_Name": name, "Grid_Size_X": grid, "Grid_Size_Y": 1, "Grid_Size_Z": 1,
                        "Start_Timestamp": start, "End_Timestamp": start + ns})  # fmt: skip


def table(out: str) -> dict[tuple[str, int], list[float]]:
    rows = {}
    for line in out.splitlines():
        parts = [p.strip() for p in line.split("|")]
        if len(parts) == 7 and parts[1].isdigit():
            rows[(parts[0], int(parts[1]))] = [float(x) for x in parts[2:]]
    return rows


def test_the_last_launches_average_is_the_timed_launches(tmp_path, capsys):
    # 5 warm-up launches of 300 us, then 4 timed ones of 100 us; written out of order, as a trace may list them.
    rows = [("k", 65536, 1_000_000 + 1000 * i, 300_000) for i in range(5)]
    rows += [("k", 65536, 2_000_000 + 1000 * i, 100_000) for i in range(4)]
    rows += [("k", 131072, 5_000_000, 50_000), ("other", 256, 6_000_000, 7_000)]
    rows.reverse()
    write_trace(tmp_path / "run_kernel_trace.csv", rows)
    bench.summarize(tmp_path, 4)
    got = table(capsys.readouterr().out)
    launches, average, last, median, least = got[("k", 65536)]
    assert launches == 9 and least == 100.0
    assert abs(average - (5 * 300 + 4 * 100) / 9) < 0.06
    assert last == 100.0  # the four latest by start time, not the four first listed
    assert median == 300.0
    assert got[("k", 131072)][:3] == [1, 50.0, 50.0]  # another grid of the same kernel is its own row


def test_the_record_reads_the_committed_traffic_line():
    t = bench.measured_traffic("cairn_wave_bf16_nn_256x256")
    assert t is not None, "profiles/traffic_wave_bf16_4096.md names the bench's bf16 kernel"
    assert t["bytes"] == t["fetch"] + t["write"]
    # Each pass reads at least the algorithmic bytes: a and b fetched once (64 MiB), c written once (32 MiB).
    assert t["fetch"] >= 2 * 4096 * 4096 * 2 and t["write"] >= 4096 * 4096 * 2
    assert bench.measured_traffic("no_such_kernel") is None
