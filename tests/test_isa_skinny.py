"""The row-streaming decode form's products on its gfx950 assembly (cairn_amd/csrc/gemm_skinny.hip, skinny_rows):
every packed dot product of a row takes its own 32-bit pair of a and of b. A bit_cast of one element of a vector
(`x[e]` of a 32-bit x 4 vector), which the kernel once used, compiled to a read of element 0 for every e: each
v_dot2 instruction then repeated four times on the same registers and the row summed a quarter of its products. The
kernel copies each element to a scalar first; this test holds the compiled code to that. No GPU is used: hipcc
cross-compiles.
"""

from __future__ import annotations

import re
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++20", "-S", "--cuda-device-only", "-ffp-contract=off",
         "-fno-fast-math", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]  # fmt: skip


@pytest.fixture(scope="module")
def rows_kernels(tmp_path_factory) -> dict[str, list[tuple[str, str]]]:
    """The v_dot2 operand pairs (a, b) of each skinny_rows instance, in program order."""
    if not shutil.which("hipcc"):
        pytest.skip("hipcc is not installed")
    out = tmp_path_factory.mktemp("isa") / "gemm_skinny.s"
    subprocess.run(["hipcc", *FLAGS, str(ROOT / "cairn_amd" / "csrc" / "gemm_skinny.hip"), "-o", str(out)], check=True,
                   capture_output=True, timeout=900)  # fmt: skip
    asm = out.read_text()
    found = {}
    for m in re.finditer(r"^(_ZN5cairn4gemm11skinny_rows\S*):", asm, re.M):
        body = asm[m.end():asm.index(".Lfunc_end", m.end())]
        dots = [line.split(";")[0].replace(",", " ").split() for line in body.splitlines() if "v_dot2" in line]
        found[m.group(1)] = [(d[2], d[3]) for d in dots]
    return found


def test_every_product_of_a_row_takes_its_own_registers(rows_kernels):
    """A row of k = 4096 is 8 pieces of 16 bytes a lane, 4 pairs each: 32 dot products for each of a's m rows, issued
    for the two rows of the loop and once more for an odd last row (96 m in all), on at least 32 m distinct register
    pairs, and never the same instruction four times running."""
    assert len(rows_kernels) == 12, sorted(rows_kernels)  # m = 1, 2; PLAIN or not; bf16, f16, f32 out
    for name, pairs in rows_kernels.items():
        m = int(re.match(r"_ZN5cairn4gemm11skinny_rowsILi(\d+)E", name).group(1))
        assert len(pairs) == 96 * m, (name, len(pairs))
        assert len(set(pairs)) >= 32 * m, (name, len(set(pairs)))
        assert not any(pairs[i] == pairs[i + 1] == pairs[i + 2] == pairs[i + 3] for i in range(len(pairs) - 3)), name
