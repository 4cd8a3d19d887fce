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
    assert t is not None, "profiles/traffic_workloads.md names the bench's bf16 kernel"
    assert t["bytes"] == t["fetch"] + t["write"]
    # Each pass reads at least the algorithmic bytes: a and b fetched once (64 MiB), c written once (32 MiB).
    assert t["fetch"] >= 2 * 4096 * 4096 * 2 and t["write"] >= 4096 * 4096 * 2
    assert bench.measured_traffic("no_such_kernel") is None


def test_blocks_times_as_the_reference_measure_does():
    """At least 2 ms a block, doubling the calls a block from 1; `count` blocks, the median of them."""
    calls = []

    def call():
        calls.append(1)
        t0 = bench.time.perf_counter()
        while bench.time.perf_counter() - t0 < 3e-4:
            pass

    t = bench.blocks(call, count=9)
    assert t["blocks"] == 9 and t["inner"] >= 4 and t["inner"] & (t["inner"] - 1) == 0  # 0.3 ms a call: 8 a block
    assert len(calls) == 1 + (2 * t["inner"] - 1) + 9 * t["inner"]  # untimed, the doublings, the blocks
    assert t["min_s"] <= t["median_s"] <= t["max_s"] and t["min_s"] >= 3e-4


def test_the_cpu_baseline_row_parallel_variant_gives_the_loop_bits():
    """cpu_baseline on tiny samples: every leg present, and the build's row-parallel variant (rows over 3 threads)
    equal bit for bit to the oracle's single-thread loop on the same inputs."""
    out = bench.cpu_baseline(n_bf16=24, n_c1=16, n_i8=16, n_rows=40, threads=3)
    assert out is not None and out["unit"] == "TFLOP/s" and out["cores"] == 1 and out["cpu"]["model"]
    assert {"c1", "int8", "row_parallel"} <= set(out)
    assert out["row_parallel"]["cores"] == 3 and "not the reference" in out["row_parallel"]["label"]
    _, port = bench.host_libraries()
    import numpy as np

    rng = np.random.default_rng(5)
    n = 37
    a = bench.bf16(rng.standard_normal((n, n), dtype=np.float32))
    b = bench.bf16(rng.standard_normal((n, n), dtype=np.float32))
    c0 = rng.standard_normal((n, n), dtype=np.float32)
    one, split = c0.copy(), c0.copy()
    P = bench.P
    assert port.oracle_mma(bench.L.BF16, n, n, n, one.ctypes.data_as(P), n * n, a.ctypes.data_as(P), n * n,
                           b.ctypes.data_as(P), n * n) == 0  # fmt: skip
    table = port.oracle_table(bench.L.BF16)
    for r0, r1 in ((0, 5), (5, 6), (6, 37)):
        port.oracle_mma_rows(bench.L.BF16, r0, r1, n, n, split.ctypes.data_as(P), a.ctypes.data_as(P),
                             b.ctypes.data_as(P), table)  # fmt: skip
    port.oracle_free(table)
    assert np.array_equal(one.view(np.uint32), split.view(np.uint32))


def test_the_counter_table_has_a_row_a_dispatch_and_a_column_a_counter(tmp_path, capsys):
    names = ["Dispatch_Id", "Kernel_Name", "Grid_Size", "Counter_Name", "Counter_Value", "Start_Timestamp",
             "End_Timestamp"]  # fmt: skip
    rows = [(1, "wave_gemm<x>(Params)", 65536, "SQ_BUSY_CYCLES", 10.0), (1, "wave_gemm<x>(Params)", 65536, "GRBM_GUI_ACTIVE", 4.0),
            (2, "copy(a)", 1024, "SQ_BUSY_CYCLES", 3.0), (1, "wave_gemm<x>(Params)", 65536, "SQ_BUSY_CYCLES", 5.0)]  # fmt: skip
    with (tmp_path / "p_counter_collection.csv").open("w", newline="") as f:
        w = csv.writer(f)
        w.writerow(names)
        for d, k, g, n, v in rows:
            w.writerow([d, k, g, n, v, 1000, 101000])
    bench.summarize(tmp_path, 1)
    out = capsys.readouterr().out.splitlines()
    assert out[0].endswith("duration us | SQ_BUSY_CYCLES | GRBM_GUI_ACTIVE")
    assert out[1] == "1 | wave_gemm<x> | 65536 | 100.0 | 15 | 4"  # a counter's instances summed
    assert out[2] == "2 | copy | 1024 | 100.0 | 3 | nan"


def test_the_cpu_leg_child_reports_its_record_or_its_end():
    """cpu_result's protocol with stand-in children: one that waits for its go and prints a record, one that aborts
    without a word (as a failed check of the reference's host code does): the bench keeps the record, or the status."""
    import subprocess

    def child(code: str) -> subprocess.Popen:
        return subprocess.Popen([sys.executable, "-c", code], stdin=subprocess.PIPE, stdout=subprocess.PIPE,
                                stderr=subprocess.PIPE, text=True)  # fmt: skip

    ok = bench.cpu_result(child("import sys, json; sys.stdin.readline(); print(json.dumps({'value': 1.5}))"))
    assert ok == {"value": 1.5}
    bad = bench.cpu_result(child("import sys, os; sys.stdin.readline(); os.abort()"))
    assert bad["error"].endswith("status -6")
