"""The tiled kernels' index arithmetic, run on the host (tests/sim/tile_sim.cpp over cairn_amd/csrc/tile.hpp and
pipe.hpp, the headers the kernels compile): in-bounds loads, every LDS chunk written once per stage, conflict-free
fragment reads on gfx950's 64 banks, every output written once, and exact products on every layout and tail. Built
under the address and undefined-behaviour sanitizers, so that a stray index in the simulation itself shows even where
the values would agree."""

from __future__ import annotations

import subprocess
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]


def test_the_tile_simulation_passes(tmp_path):
    exe = tmp_path / "tile_sim"
    subprocess.run(["g++", "-std=c++20", "-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=all",
                    "-Wall", "-Wextra", "-Werror", "-Wno-unknown-pragmas", f"-I{ROOT / 'cairn_amd' / 'csrc'}",
                    str(ROOT / "tests" / "sim" / "tile_sim.cpp"), "-o", str(exe)], check=True)  # fmt: skip
    done = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600)
    assert done.returncode == 0 and "Sanitizer" not in done.stderr, done.stdout[-3000:] + done.stderr[-3000:]
    assert done.stdout.strip().endswith("ok: every tile equals the exact product"), done.stdout[-3000:]
