"""What the one-wave-a-SIMD kernel (cairn_amd/csrc/wave.hpp, instances in gemm_wave_<type>.hip) needs of the compiler, checked on its gfx950
assembly: M0 holds the LDS base of a group of loads and each load picks its KiB by immediate offset, so between a write
of M0 and the loads of its group nothing may write M0 again. The kernel writes M0 in inline assembly the compiler
cannot see into; this test reads what the compiler emitted and holds it to that. No GPU is used: hipcc cross-compiles.
"""

from __future__ import annotations

import concurrent.futures
import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++20", "-S", "--cuda-device-only", "-ffp-contract=off",
         "-fno-fast-math", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]  # fmt: skip


@pytest.fixture(scope="module")
def assembly(tmp_path_factory) -> str:
    if not shutil.which("hipcc"):
        pytest.skip("hipcc is not installed")
    where = tmp_path_factory.mktemp("isa")

    def compiled(src: Path) -> str:
        out = where / (src.stem + ".s")
        subprocess.run(["hipcc", *FLAGS, str(src), "-o", str(out)], check=True, capture_output=True, timeout=900)
        return out.read_text()

    with concurrent.futures.ThreadPoolExecutor(4) as pool:
        return "\n".join(pool.map(compiled, sorted((ROOT / "cairn_amd" / "csrc").glob("gemm_wave_*.hip"))))


def kernels(asm: str) -> dict[str, list[str]]:
    found = {}
    for m in re.finditer(r"^(_ZN5cairn4gemm(?:9wave_gemm|10wave8_gemm|10wave_split|11wave8_split)\S*):", asm, re.M):
        body = asm[m.end():asm.index(".Lfunc_end", m.end())]
        found[m.group(1)] = [line.split(";")[0].strip() for line in body.splitlines() if line.strip()]
    return found


def test_every_lds_load_group_starts_with_its_own_base(assembly):
    ks = kernels(assembly)
    assert len(ks) >= 40  # the whole-tile and split kernels of every instance
    for name, lines in ks.items():
        groups, current = [], None
        for line in lines:
            if "m0" in line:
                assert re.fullmatch(r"s_mov_b32 m0, s\d+", line), (name, line)  # only the kernel's own writes
                current = []
                groups.append(current)
            elif re.match(r"buffer_load_dwordx4 .* lds$", line):
                assert current is not None, (name, "an LDS load before any base", line)
                offset = re.search(r"offset:(0x[0-9a-f]+|\d+)", line)
                current.append(int(offset.group(1), 0) if offset else 0)
        assert groups, name
        for g in groups:
            assert g == [1024 * u for u in range(len(g))] and 1 <= len(g) <= 4, (name, g)


def test_the_main_loop_writes_m0_twice_per_stage(assembly):
    for name, lines in kernels(assembly).items():
        loops = []
        for i, line in enumerate(lines):
            if re.match(r"s_cbranch_scc[01] (\.LBB\S+)", line):
                target = line.split()[-1]
                start = lines.index(target + ":")
                if start < i and any("s_barrier" in x for x in lines[start:i]):
                    loops.append(lines[start:i])
        assert loops, name
        loop = max(loops, key=lambda seg: sum(x.startswith("v_mfma") for x in seg))  # the main loop
        fp8 = "wave8_" in name  # one 32x32x64 MFMA a block and stage; the int8 layout's two k-steps otherwise
        mfmas = sum(x.startswith("v_mfma") for x in loop)
        stages = mfmas // (16 if fp8 else 32)
        # Every steady loop is unrolled by the ring's four stages.
        assert stages == 4 and mfmas == stages * (16 if fp8 else 32), (name, mfmas)
        assert sum("m0" in x for x in loop) == 2 * stages, name
        assert sum(x == "s_barrier" for x in loop) == stages, name
        assert not any(x.startswith(("scratch_", "buffer_store")) for x in loop), name  # no spills in the loop


def issue_cycles(loop: list[str], mfma: int = 32) -> tuple[int, int]:
    """A static price of a loop for one wave alone on its SIMD: the wave issues one instruction every 4 cycles, and
    an MFMA at most every `mfma` cycles (32 for a 32 x 32 bf16 / int8 MFMA's passes, 64 for the 32 x 32 x 64 fp8
    one), so the instructions between two MFMAs cost time only past mfma / 4 - 1. Returns (cycles, the MFMAs' own
    cycles)."""
    gaps, cur = [], 0
    for x in loop:
        if not x or x.endswith(":"):
            continue
        op = x.split()[0]
        if op.startswith("v_mfma"):
            gaps.append(cur)
            cur = 0
        else:
            cur += 1 + (int(x.split()[1]) if op == "s_nop" else 0)
    gaps[0] += cur  # the loop wraps around
    return sum(max(mfma, 4 * (g + 1)) for g in gaps), mfma * len(gaps)


def test_the_steady_loop_issues_in_the_mfmas_shadow(assembly):
    """Between two MFMAs a lone wave has seven issue slots (fifteen for fp8); the steady loop's reads, loads, waits and
    scalar work (the walked buffer resources, placed in slots no read or load uses) fit in them: the static price is
    within 1% of the MFMAs' own time for every kernel."""
    for name, lines in kernels(assembly).items():
        loops = []
        for i, line in enumerate(lines):
            if re.match(r"s_cbranch_scc[01] (\.LBB\S+)", line):
                start = lines.index(line.split()[-1] + ":")
                if start < i and any("s_barrier" in x for x in lines[start:i]):
                    loops.append(lines[start:i + 1])
        loop = max(loops, key=lambda seg: sum(x.startswith("v_mfma") for x in seg))
        cycles, ideal = issue_cycles(loop, 64 if "wave8_" in name else 32)
        assert cycles <= 1.01 * ideal, (name, cycles, ideal)
