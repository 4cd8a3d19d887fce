"""The tiled kernels' index arithmetic, run on the host (tests/sim/tile_sim.cpp over cairn_amd/csrc/tile.hpp and
pipe.hpp, the headers the kernels compile): in-bounds loads, every LDS chunk written once per stage, conflict-free
fragment reads on gfx950's 64 banks, every output written once, and exact products on every layout and tail."""

from __future__ import annotations

import subprocess
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def test_the_tile_simulation_passes(tmp_path):
    exe = tmp_path / "tile_sim"
    subprocess.run(["g++", "-std=c++20", "-O2", "-Wall", "-Wextra", "-Werror", "-Wno-unknown-pragmas",
                    f"-I{ROOT / 'cairn_amd' / 'csrc'}", str(ROOT / "tests" / "sim" / "tile_sim.cpp"), "-o", str(exe)],
                   check=True)  # fmt: skip
    done = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert done.returncode == 0, done.stdout[-3000:]
    assert done.stdout.strip().endswith("ok: every tile equals the exact product"), done.stdout[-3000:]
