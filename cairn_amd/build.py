"""Build libcairn_gemm_gfx950.so in-tree: every HIP and C++ source under cairn_amd/csrc compiled by hipcc for gfx950,
then linked into one shared library beside this file.

Device and host code both build with -ffp-contract=off: the epilogue's steps are each an f32 rounding in the order
include/cairn_gemm.h states (no fused multiply-add folds a scale into a bias), and the host reference loop of the C++
surface keeps the reference's rounding (src/cairn/projects/toolchain.py:29-30). Every HIP compile also turns off the
packed-fp32 instruction feature, so no v_pk_{add,mul,fma}_f32 is ever emitted.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
from pathlib import Path

from cairn_amd import identity

HERE = Path(__file__).resolve().parent
SOURCES = HERE / "csrc"
OBJECTS = HERE / "_build"
LIBRARY = HERE / "libcairn_gemm_gfx950.so"
ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

COMMON = ["-O3", "-std=c++20", "-fPIC", "-ffp-contract=off", "-fno-fast-math", "-Wall", "-Wno-unused-parameter",
          "-fno-exceptions", "-fno-rtti"]  # fmt: skip
DEVICE = [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]


def sources() -> list[Path]:
    return sorted([*SOURCES.glob("*.hip"), *SOURCES.glob("*.cpp")])


def _compile(src: Path) -> tuple[Path, str]:
    obj = OBJECTS / (src.name + ".o")
    cmd = [HIPCC, *DEVICE, *COMMON, "-c", str(src), "-o", str(obj)]
    done = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"  # the host pass does not know the device feature
    err = "\n".join(line for line in done.stderr.splitlines() if noise not in line)
    if done.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{err[-6000:]}")
    return obj, err


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every source and link the library; returns its path. Always rebuilds."""
    if not shutil.which(HIPCC) and not Path(HIPCC).exists():
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    identity.check()  # the header's interface identity is the hash of what it states
    OBJECTS.mkdir(exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), os.cpu_count() or 4, 16)
    with concurrent.futures.ThreadPoolExecutor(jobs) as pool:
        results = list(pool.map(_compile, srcs))
    for obj, err in results:
        if verbose and err.strip():
            print(err)
    tmp = LIBRARY.with_suffix(".so.tmp")
    link = [HIPCC, *DEVICE, "-shared", "-fPIC", *[str(o) for o, _ in results], "-o", str(tmp)]
    done = subprocess.run(link, capture_output=True, text=True)
    if done.returncode != 0:
        raise RuntimeError(f"link failed:\n{done.stderr[-6000:]}")
    tmp.replace(LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    print(build(verbose=True))
