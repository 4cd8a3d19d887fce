"""The MFMA fragments' host model (include/cairn/cairn_fragment.hpp) on the CPU: tests/cpp/fragment_host.cpp runs one
wave of 64 host threads through every shape and operand type, under the thread sanitizer, and checks the results
against the reference loop bit for bit, that each element is written once by the lane the device gives it, and that
get/set name a lane's own elements. An index past a lane's share must abort the process, as the reference's trap
does (src/cairn/runtime/cairn_fragment.hpp:254-276)."""

from __future__ import annotations

import signal
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


@pytest.fixture(scope="module")
def program(tmp_path_factory) -> Path:
    exe = tmp_path_factory.mktemp("frag") / "fragment_host"
    subprocess.run(["g++", "-std=c++20", "-O1", "-g", "-ffp-contract=off", "-fsanitize=thread", "-pthread",
                    f"-I{ROOT / 'include' / 'cairn'}", str(ROOT / "tests" / "cpp" / "fragment_host.cpp"), "-o",
                    str(exe)], check=True, capture_output=True, timeout=300)  # fmt: skip
    return exe


def test_every_lane_equals_the_reference_and_writes_its_own_elements_once(program):
    done = subprocess.run([str(program)], capture_output=True, text=True, timeout=300)
    assert done.returncode == 0, done.stdout + done.stderr
    assert "every lane's fragments equal the reference" in done.stdout
    assert done.stdout.count("ok ") == 7 and "WARNING: ThreadSanitizer" not in done.stderr


def test_an_index_past_the_share_aborts(program):
    done = subprocess.run([str(program), "trap"], capture_output=True, text=True, timeout=120)
    assert done.returncode == -signal.SIGABRT
