"""The C++ surface in include/cairn, built with g++ on the host under the address and undefined-behaviour sanitizers:
tests/cpp/surface.cpp under a recording machine (the execution context's rules, its traps, and the storage floats and
host multiply bit for bit against the reference's own outputs, tests/golden/reference.npz), and tests/cpp/emitted.cpp,
an emitted-shaped unit, linked against the library and built emulated (-DCAIRN_EMULATE) and run."""

from __future__ import annotations

import subprocess
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
GOLDEN = np.load(ROOT / "tests" / "golden" / "reference.npz")
FORMATS = ["f16", "bf16", "f8e4m3", "f8e5m2"]
SANITIZED = ["-O1", "-g", "-fsanitize=address,undefined", "-fno-sanitize-recover=all"]


@pytest.fixture(scope="module")
def surface(tmp_path_factory) -> Path:
    exe = tmp_path_factory.mktemp("surface") / "surface"
    subprocess.run(["g++", "-std=c++20", *SANITIZED, "-ffp-contract=off", "-Wall", "-Wextra", "-Werror",
                    "-DCAIRN_GEMM_UNLINKED=1", f"-I{ROOT / 'include'}", str(ROOT / "tests" / "cpp" / "surface.cpp"),
                    "-o", str(exe)], check=True)  # fmt: skip
    return exe


def run(exe: Path, *args: str) -> subprocess.CompletedProcess:
    return subprocess.run([str(exe), *args], capture_output=True, text=True, timeout=60)


def test_the_context_keeps_the_reference_rules(surface):
    done = run(surface, "context")
    assert done.returncode == 0 and "Sanitizer" not in done.stderr, done.stdout + done.stderr
    lines = done.stdout.splitlines()
    assert lines[-1] == "0 failures" and sum(line.startswith("ok ") for line in lines) >= 40


@pytest.mark.parametrize("case", ["shape", "nested", "settle", "observe", "leaked", "lease", "unleased", "ticket",
                                  "rebind", "overflow", "e4m3", "scale"])
def test_misuse_traps(surface, case):
    done = run(surface, "trap", case)
    assert done.returncode == -6 and "returned" not in done.stdout, (done.returncode, done.stdout)


@pytest.mark.parametrize("fmt", FORMATS)
def test_storage_floats_match_the_reference(surface, fmt, tmp_path):
    x = GOLDEN[f"narrow_{fmt}_x"]
    x.astype(np.float64).tofile(tmp_path / "x")
    assert run(surface, "narrow", fmt, str(tmp_path / "x"), str(tmp_path / "y")).returncode == 0
    assert np.array_equal(np.fromfile(tmp_path / "y", np.uint32), GOLDEN[f"narrow_{fmt}_bits"])

    q = np.stack([GOLDEN[f"quantize_{fmt}_x"], GOLDEN[f"quantize_{fmt}_scale"]], axis=1).astype(np.float32)
    q.tofile(tmp_path / "q")
    assert run(surface, "quantize", fmt, str(tmp_path / "q"), str(tmp_path / "r")).returncode == 0
    assert np.array_equal(np.fromfile(tmp_path / "r", np.uint32), GOLDEN[f"quantize_{fmt}_bits"])

    GOLDEN[f"decode_{fmt}_bits"].astype(np.uint32).tofile(tmp_path / "p")
    assert run(surface, "decode", fmt, str(tmp_path / "p"), str(tmp_path / "v")).returncode == 0
    got, want = np.fromfile(tmp_path / "v", np.float64), GOLDEN[f"decode_{fmt}_value"]
    assert np.array_equal(got.view(np.uint64), want.view(np.uint64))  # NaN payloads and signed zeros included


@pytest.mark.parametrize("fmt", FORMATS)
def test_the_host_multiply_is_the_reference_loop(surface, fmt, tmp_path):
    keys = sorted({k.rsplit("_", 1)[0] for k in GOLDEN.files if k.startswith((f"mma_{fmt}_", f"tile_{fmt}_"))})
    if fmt == "f16":
        keys += ["app_layer", "app_order"]
    assert len(keys) >= 14
    for key in keys:
        m, n, k = (int(v) for v in GOLDEN[key + "_shape"])
        for part in ("a", "b", "c"):
            GOLDEN[f"{key}_{part}"].tofile(tmp_path / part)
        done = run(surface, "mma", fmt, str(m), str(n), str(k), *(str(tmp_path / p) for p in ("a", "b", "c")),
                   str(tmp_path / "out"))  # fmt: skip
        assert done.returncode == 0, (key, done.stderr)
        got = np.fromfile(tmp_path / "out", np.float32)
        assert np.array_equal(got.view(np.uint32), GOLDEN[key + "_out"].view(np.uint32)), key


def test_emitted_code_builds_against_the_include_set_and_the_library(tmp_path):
    """An emitted-shaped unit (tests/cpp/emitted.cpp) compiles with g++ on include/cairn alone and links against the
    library: the spellings emitted code uses (cr::tensor::launch, cr::gpu::here, cr::view, cr::disjoint,
    cr::gpu::Enqueued, the storage floats) all resolve."""
    from cairn_amd import lib as L

    L.load()
    rocm = Path("/opt/rocm")
    exe = tmp_path / "emitted"
    subprocess.run(["g++", "-std=c++20", "-O2", "-ffp-contract=off", "-fno-exceptions", "-fno-rtti", "-Wall", "-Wextra",
                    "-Werror", "-D__HIP_PLATFORM_AMD__", f"-I{ROOT / 'include' / 'cairn'}", f"-I{rocm / 'include'}",
                    str(ROOT / "tests" / "cpp" / "emitted.cpp"), "-o", str(exe), f"-L{L.LIBRARY.parent}",
                    f"-l:{L.LIBRARY.name}", f"-L{rocm / 'lib'}", "-lamdhip64", f"-Wl,-rpath,{L.LIBRARY.parent}"],
                   check=True)  # fmt: skip
    syms = subprocess.run(["nm", str(exe)], capture_output=True, text=True, check=True).stdout
    assert "cf_emitted_mma" in syms and "cq_emitted_mma" in syms
    assert "cairn_gemm_mma" in subprocess.run(["nm", "-u", str(exe)], capture_output=True, text=True).stdout


def test_emitted_code_runs_emulated_as_the_host_multiply(tmp_path):
    """`cairn build --emulate` (src/cairn/projects/toolchain.py:175-180): the emitted-shaped unit built by the host
    compiler with -DCAIRN_EMULATE, no library and no GPU. launch<A> on the emulated machine is the host loop
    (src/cairn/runtime/cairn_emulate.hpp:151-156), bit for bit, for every storage float on the reference's device
    shapes; the C entries run held and enqueued; a descriptor's GEMM follows its stated steps."""
    exe = tmp_path / "emulated"
    subprocess.run(["g++", "-std=c++20", *SANITIZED, "-ffp-contract=off", "-fno-exceptions", "-fno-rtti", "-Wall",
                    "-Wextra", "-Werror", "-DCAIRN_EMULATE", f"-I{ROOT / 'include' / 'cairn'}",
                    str(ROOT / "tests" / "cpp" / "emitted.cpp"), "-o", str(exe)], check=True)  # fmt: skip
    assert "cairn_gemm" not in subprocess.run(["nm", "-u", str(exe)], capture_output=True, text=True).stdout
    done = run(exe)
    assert done.returncode == 0 and "Sanitizer" not in done.stderr, done.stdout + done.stderr
    lines = done.stdout.splitlines()
    assert lines[-1] == "0 failures" and sum(line.startswith("ok ") for line in lines) == 6
