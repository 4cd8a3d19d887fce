"""The device quantize (cairn_quantize_run, cairn_amd/csrc/quantize.hip) on the CPU: its element arithmetic against the
reference's quantize, the oracle's row contract against the element function and numpy, and the entry's refusals.

- The kernel decides most elements with an f32 shortcut and the rest with the reference's double steps
  (src/cairn/runtime/cairn_float.hpp:116-146). tests/cpp/quantize_shortcut.cpp compiles that same header for the host
  and drives it through every rounding boundary of int8, E4M3 and E5M2 at many scales, against the oracle.
- oracle_quantize_rows (the GPU tests' checker) is the element function applied row by row, with the computed scale
  being numpy's largest |x| of the row over the format's range in f32.
- cairn_quantize_run refuses bad descriptors before any HIP call, so those run here without a GPU.
"""

from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np
import pytest

import helpers as H
from cairn_amd import lib as L

ROOT = Path(__file__).resolve().parents[1]
RANGE = {L.I8: 127.0, L.F8E4M3: 448.0, L.F8E5M2: 57344.0}


def test_the_shortcut_equals_the_reference_quantize_at_every_boundary(tmp_path):
    obj = tmp_path / "oracle.o"
    exe = tmp_path / "shortcut"
    flags = ["-O2", "-ffp-contract=off", "-fno-fast-math"]
    subprocess.run(["gcc", *flags, "-std=c11", "-c", str(ROOT / "oracle" / "oracle.c"), "-o", str(obj)], check=True)
    subprocess.run(["g++", *flags, "-std=c++20", f"-I{ROOT / 'cairn_amd' / 'csrc'}",
                    str(ROOT / "tests" / "cpp" / "quantize_shortcut.cpp"), str(obj), "-lm", "-o", str(exe)],
                   check=True)  # fmt: skip
    done = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert done.returncode == 0, done.stdout + done.stderr
    words = done.stdout.split()
    checked, decided, declined = int(words[1]), int(words[3]), int(words[5])
    assert checked > 5_000_000 and decided > checked // 2 and declined > 100_000, done.stdout


def element(q_type: int, x: float, s: float) -> tuple[int, bool]:
    o, t = H.oracle(), C.c_int()
    if q_type == L.I8:
        v = o.oracle_quantize_int(x, s, -128, 127, C.byref(t))
        return (0 if t.value else v) & 0xFF, bool(t.value)
    return o.oracle_quantize_float(q_type, x, s, C.byref(t)), bool(t.value)


@pytest.mark.parametrize("q_type", [L.I8, L.F8E4M3, L.F8E5M2])
def test_the_rows_oracle_is_the_element_function_with_numpy_scales(q_type):
    rng = np.random.default_rng(5 + q_type)
    m, k = 9, 37
    x = (rng.standard_normal((m, k)) * np.logspace(-3, 3, m)[:, None]).astype(np.float32)
    x[1] = 0.0                         # a zero row: scale 1, every output 0
    x[2, 3] = np.nan                   # NaN left out of the largest magnitude
    x[3, 5] = np.inf                   # an infinite row: the reference traps on its scale
    x[4, :4] = [-0.0, 1e-45, -3e38, 3e38]
    q, s, status = H.quantize_rows(L.F32, q_type, L.SCALE_ROW_ABSMAX, x, k)
    with np.errstate(invalid="ignore"):
        top = np.nanmax(np.abs(x), axis=1).astype(np.float32)
    want_s = np.where(top == 0, np.float32(1), top / np.float32(RANGE[q_type])).astype(np.float32)
    assert np.array_equal(s.view(np.uint32), want_s.view(np.uint32))
    trap = 0
    for i in range(m):
        for j in range(k):
            if not (0 < want_s[i] < np.inf):
                assert q[i, j] == 0
                continue
            v, t = element(q_type, float(x[i, j]), float(want_s[i]))
            trap |= t
            assert q[i, j] == v, (i, j)
    assert status == (L.QUANT_BAD_SCALE | (L.QUANT_NAN if q_type == L.I8 else 0))
    # Given scales: per row, and one for the whole matrix.
    given = np.linspace(0.01, 2.0, m).astype(np.float32)
    q2, _, _ = H.quantize_rows(L.F32, q_type, L.SCALE_ROW, x, k, given)
    q3, _, _ = H.quantize_rows(L.F32, q_type, L.SCALE_TENSOR, x, k, given[:1])
    for i in (0, 5, 8):
        for j in range(0, k, 5):
            assert q2[i, j] == element(q_type, float(x[i, j]), float(given[i]))[0]
            assert q3[i, j] == element(q_type, float(x[i, j]), float(given[0]))[0]


def test_the_rows_oracle_reads_16_bit_inputs_exactly():
    rng = np.random.default_rng(3)
    xf = rng.standard_normal((4, 24)).astype(np.float32)
    xb = H.bf16_from_f32(xf)
    q_b, s_b, _ = H.quantize_rows(L.BF16, L.I8, L.SCALE_ROW_ABSMAX, xb, 24)
    q_f, s_f, _ = H.quantize_rows(L.F32, L.I8, L.SCALE_ROW_ABSMAX, H.f32_from_bf16(xb), 24)
    assert np.array_equal(q_b, q_f) and np.array_equal(s_b, s_f)
    xh = xf.astype(np.float16).view(np.uint16)
    q_h, _, _ = H.quantize_rows(L.F16, L.F8E4M3, L.SCALE_ROW_ABSMAX, xh, 24)
    q_g, _, _ = H.quantize_rows(L.F32, L.F8E4M3, L.SCALE_ROW_ABSMAX, H.f32_from_f16(xh), 24)
    assert np.array_equal(q_h, q_g)


def test_the_documented_answers():
    # docs/numerics.md:32 of the reference: quantize[i8](-2.5, 1.0) == -2, quantize[i8](500.0, 2.0) == 127.
    x = np.array([[-2.5, 250.0, 0.5, 1.5]], dtype=np.float32)  # ties to even; saturation
    q, _, _ = H.quantize_rows(L.F32, L.I8, L.SCALE_TENSOR, x, 4, np.array([1.0], np.float32))
    assert q.view(np.int8).tolist() == [[-2, 127, 0, 2]]
    q, _, _ = H.quantize_rows(L.F32, L.I8, L.SCALE_TENSOR, np.array([[500.0]], np.float32), 1,
                              np.array([2.0], np.float32))  # fmt: skip
    assert q.view(np.int8).tolist() == [[127]]


def test_the_entry_refuses_bad_descriptors_before_any_gpu_call():
    lib = L.load()
    P = 1 << 20

    def status(**kw) -> int:
        args = dict(x_type=L.BF16, q_type=L.I8, m=4, k=16, x=P, q=P, scale=P)
        args.update(kw)
        d = L.quantize_desc(args.pop("x_type"), args.pop("q_type"), args.pop("m"), args.pop("k"), args.pop("x"),
                            args.pop("q"), args.pop("scale"), **args)  # fmt: skip
        return lib.cairn_quantize_run(C.byref(d), None)

    assert status(q_type=L.F16) == L.E_TYPE and status(x_type=L.I8) == L.E_TYPE
    assert status(mode=7) == L.E_ARG and status(scale=None) == L.E_ARG and status(x=None) == L.E_ARG
    assert status(ldx=8) == L.E_SHAPE and status(ldq=3) == L.E_SHAPE and status(m=1 << 31) == L.E_SHAPE
    assert status(k=(1 << 28) + 8, ldx=0, ldq=0) == L.E_SHAPE
    assert status(m=0) == L.OK  # nothing to do: no launch
    d = L.quantize_desc(L.BF16, L.I8, 4, 16, P, P, P)
    d.version = 9
    assert lib.cairn_quantize_run(C.byref(d), None) == L.E_ARG
