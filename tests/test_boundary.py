"""The drop-in boundary on the CPU: libcairn_gemm_gfx950.so loads and exports every symbol include/cairn_gemm.h
declares, its structs have the layout the header states, the host entries (cf_mma_<fmt>: the reference loop) equal
the oracle bit for bit, the checked entries abort where the reference traps, and the selector answers for every
BASELINE config and refuses what no kernel computes. No test here launches GPU work.
"""

from __future__ import annotations

import ctypes as C
import hashlib
import re
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

import helpers as H
from cairn_amd import identity
from cairn_amd import lib as L

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "cairn_gemm.h"


def declared_functions() -> set[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    names = set(re.findall(r"^(?:[A-Za-z_][\w\s\*]*?)\b([A-Za-z_]\w*)\s*\([^;]*\)\s*;", text, flags=re.M))
    return {n for n in names if n not in {"typedef"}}


def test_the_library_exports_every_declared_symbol():
    L.load()
    names = declared_functions()
    assert {"cairn_gemm_run", "cairn_gemm_select", "cf_mma_bf16", "cq_mma_bf16_device", "cairn_gemm_device_stream"} <= names
    dynamic = subprocess.run(["nm", "-D", "--defined-only", str(L.LIBRARY)], capture_output=True, text=True,
                             check=True).stdout  # fmt: skip
    exported = {line.split()[-1] for line in dynamic.splitlines() if len(line.split()) >= 3}
    missing = (names | set(L.DATA_SYMBOLS)) - exported
    assert not missing, missing
    assert names == set(L.SIGNATURES), names ^ set(L.SIGNATURES)  # the bindings type every entry
    lib = L.load()
    assert (C.c_char * 12).in_dll(lib, L.DATA_SYMBOLS[0]).value == b"gemm_gfx950"


def test_the_interface_identity_is_the_hash_of_the_stated_interface():
    """header.py:280-285: cairn_interface_<library>_<sha256 of the stated interface, 16 hex digits>. The header's line
    is the hash of its own stated text, the library defines exactly that symbol, and a change to any declaration
    changes it."""
    text = HEADER.read_text()
    stated = identity.stated(text)
    assert "int cairn_gemm_run(" in stated and "cairn_quantize_desc" in stated
    assert identity.declared(text) == identity.check()
    assert identity.derived(text) == "cairn_interface_gemm_gfx950_" + hashlib.sha256(stated.encode()).hexdigest()[:16]
    edited = text.replace("int cairn_gemm_run(const cairn_gemm_desc* d, void* stream);",
                          "int cairn_gemm_run(const cairn_gemm_desc* d, void* stream, int flags);")  # fmt: skip
    assert edited != text and identity.derived(edited) != identity.derived(text)
    dynamic = subprocess.run(["nm", "-D", "--defined-only", str(L.LIBRARY)], capture_output=True, text=True,
                             check=True).stdout  # fmt: skip
    ids = {line.split()[-1] for line in dynamic.splitlines() if "cairn_interface_" in line}
    assert ids == {identity.declared(text)}
    assert (C.c_char * 12).in_dll(L.load(), identity.declared(text)).value == b"gemm_gfx950"  # a char array


def test_a_program_built_against_another_version_of_the_header_fails_to_link(tmp_path):
    """The header refers to its identity, so a program that includes it needs the library of the same stated
    interface: against this header it links; against a copy whose run entry gained a parameter (and so a new
    identity, written as identity.py writes it) the link fails on that identity's symbol."""
    src = tmp_path / "caller.c"
    src.write_text('#include "cairn_gemm.h"\nint main(void) { return cairn_gemm_kernel_count() > 0 ? 0 : 1; }\n')
    def link(include: Path) -> subprocess.CompletedProcess:
        return subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", f"-I{include}", str(src), "-o",
                               str(tmp_path / "caller"), f"-L{L.LIBRARY.parent}", f"-l:{L.LIBRARY.name}",
                               f"-Wl,-rpath,{L.LIBRARY.parent}"], capture_output=True, text=True)  # fmt: skip
    assert link(HEADER.parent).returncode == 0
    stale = tmp_path / "stale"
    stale.mkdir()
    text = HEADER.read_text().replace("int cairn_gemm_run(const cairn_gemm_desc* d, void* stream);",
                                      "int cairn_gemm_run(const cairn_gemm_desc* d, void* stream, int flags);")
    other = identity.derived(text)
    (stale / "cairn_gemm.h").write_text(identity.DEFINE.sub(f"#define CAIRN_GEMM_IDENTITY {other}", text))
    done = link(stale)
    assert done.returncode != 0 and other in done.stderr, done.stderr


def test_the_structs_have_the_layout_the_header_states(tmp_path):
    structs = {"cairn_gemm_desc": L.Desc, "cairn_gemm_kernel": L.Kernel, "cairn_gemm_choice": L.Choice,
               "cairn_quantize_desc": L.QuantizeDesc}  # fmt: skip
    fields = {name: [f for f, _ in cls._fields_] for name, cls in structs.items()}
    lines = ["#include <stdio.h>", "#include <stddef.h>", "#define CAIRN_GEMM_UNLINKED 1", f'#include "{HEADER}"',
             "int main(void) {"]  # the layouts only: no library to link
    for struct, names in fields.items():
        lines.append(f'printf("{struct} %zu\\n", sizeof({struct}));')
        lines += [f'printf("{struct}.{f} %zu\\n", offsetof({struct}, {f}));' for f in names]
    lines += ["return 0;", "}"]
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", str(src), "-o", str(exe)], check=True)
    got = dict(line.rsplit(" ", 1) for line in subprocess.run([str(exe)], capture_output=True, text=True,
                                                              check=True).stdout.splitlines())  # fmt: skip
    for struct, cls in structs.items():
        assert int(got[struct]) == C.sizeof(cls), struct
        for f in fields[struct]:
            assert int(got[f"{struct}.{f}"]) == getattr(cls, f).offset, (struct, f)


@pytest.mark.parametrize("name", ["f32", "f16", "bf16", "f8e4m3", "f8e5m2"])
def test_the_host_entries_are_the_reference_loop(name):
    fmt = {"f32": H.F32, "f16": H.F16, "bf16": H.BF16, "f8e4m3": H.F8E4M3, "f8e5m2": H.F8E5M2}[name]
    rng = np.random.default_rng(17)
    f = getattr(L.load(), f"cf_mma_{name}")
    for m, n, k in [(1, 1, 1), (17, 3, 33), (12, 13, 64), (40, 41, 7), (3, 4, 0)]:
        if fmt == H.F32:
            a = rng.uniform(-1, 1, m * k).astype(np.float32)
            b = rng.uniform(-1, 1, k * n).astype(np.float32)
        else:
            a = H.encode(fmt, np.round(rng.uniform(-8, 8, m * k) * 8) / 8)
            b = H.encode(fmt, np.round(rng.uniform(-8, 8, k * n) * 8) / 8)
        c = rng.uniform(-4, 4, m * n).astype(np.float32)
        want = c.copy()
        assert H.mma(fmt, m, n, k, want, a, b) == 0
        got = c.copy()
        f(m, n, k, got.size, got.ctypes.data, a.size, a.ctypes.data, b.size, b.ctypes.data)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (name, m, n, k)


ABORT = """
import ctypes as C, numpy as np, sys
sys.path.insert(0, {root!r})
from cairn_amd import lib as L
f = L.load().cf_mma_bf16
a = np.zeros(6, np.uint16); b = np.zeros(9, np.uint16); c = np.zeros(6, np.float32)
{call}
print("returned")
"""


@pytest.mark.parametrize("call", [
    "f(2, 3, 3, 6, c.ctypes.data, 6, a.ctypes.data, 6, b.ctypes.data)",   # b holds 9, the call says 6
    "f(2, 3, 3, 5, c.ctypes.data, 6, a.ctypes.data, 9, b.ctypes.data)",   # c holds 6, the call says 5
    "f(2, 3, 3, 6, c.ctypes.data, 6, c.ctypes.data, 9, b.ctypes.data)",   # a overlaps the read-write c
    "f(2, 3, 3, 6, None, 6, a.ctypes.data, 9, b.ctypes.data)",            # a null view of 6 elements
])  # fmt: skip
def test_the_checked_entry_aborts_where_the_reference_traps(call):
    """src/cairn/runtime/cairn_tensor.hpp:22-24 (shape), codegen.py:500-512 (views, disjoint): a failed check is
    std::abort, SIGABRT, never a return (tests/soundness/test_tensor.py:109-119)."""
    done = subprocess.run([sys.executable, "-c", ABORT.format(root=str(ROOT), call=call)], capture_output=True,
                          text=True, timeout=120)  # fmt: skip
    assert done.returncode == -6, (done.returncode, done.stdout, done.stderr[-500:])
    assert "returned" not in done.stdout


def test_a_and_b_may_be_one_array():
    """test_tensor.py:105-106: a square of one matrix reads it twice."""
    f = L.load().cf_mma_bf16
    a = H.encode(H.BF16, np.arange(9, dtype=np.float64) / 8)
    c = np.zeros(9, np.float32)
    f(3, 3, 3, 9, c.ctypes.data, 9, a.ctypes.data, 9, a.ctypes.data)
    want = np.zeros(9, np.float32)
    H.mma(H.BF16, 3, 3, 3, want, a, a)
    assert np.array_equal(c, want)


# ------------------------------------------------------------------ the selector


P = 1 << 20  # an aligned stand-in address: select only reads pointer alignment


def choose(*args, **kw):
    return L.select(L.desc(*args, **kw))


def test_the_selector_picks_a_kernel_for_every_baseline_config():
    c2 = choose(L.BF16, L.BF16, 4096, 4096, 4096, P, P, P)
    assert c2["family"] == "wave" and (c2["tile_m"], c2["tile_n"]) == (256, 256) and c2["workgroups"] == 256
    c4 = choose(L.I8, L.BF16, 4096, 4096, 4096, P, P, P, row_scale=P, col_scale=P)
    assert c4["family"] == "wave" and "i8" in c4["name"]
    assert choose(L.I8, L.I32, 4096, 4096, 4096, P, P, P)["family"] == "wave"
    for m in (1, 4, 16):
        assert choose(L.BF16, L.BF16, m, 14336, 4096, P, P, P, trans_b=True)["family"] == "skinny"
    fwd = choose(L.BF16, L.BF16, 8192, 11008, 4096, P, P, P, bias=P, bias_type=L.BF16, act=L.ACT_GELU)
    dx = choose(L.BF16, L.BF16, 8192, 4096, 11008, P, P, P, trans_b=True)
    dw = choose(L.BF16, L.BF16, 4096, 11008, 8192, P, P, P, trans_a=True)
    assert [x["name"].split("_")[3] for x in (fwd, dx, dw)] == ["nn", "nt", "tn"]
    assert fwd["waves"] == pytest.approx(1376 / 256) and dx["workgroups"] == 512


def test_the_selector_falls_back_to_the_generic_kernel_where_chunks_do_not_fit():
    assert choose(L.BF16, L.F32, 65, 63, 33, P, P, P, accumulate=True)["family"] == "generic"  # k % 8
    assert choose(L.F8E4M3, L.F32, 200, 136, 68, P, P, P, accumulate=True)["family"] == "generic"  # k % 8
    assert choose(L.F8E4M3, L.F32, 200, 132, 72, P, P, P, accumulate=True)["family"] == "generic"  # n % 8 (NN's b)
    # The 8-bit floats go to the MFMA kernel, which widens them to f16 (8-byte pieces: 72 of k is enough); the ring's
    # 8-bit float matrix core runs where it is named.
    assert choose(L.F8E4M3, L.F32, 200, 136, 72, P, P, P, accumulate=True)["name"] == "cairn_mfma_f8e4m3_nn_128x128"
    f8 = choose(L.F8E5M2, L.F32, 256, 256, 256, P, P, P, accumulate=True)
    assert f8["family"] == "mfma" and f8["name"] == "cairn_mfma_f8e5m2_nn_128x128" and f8["tile_k"] == 64
    named = choose(L.F8E5M2, L.F32, 256, 256, 256, P, P, P, accumulate=True,
                   kernel=L.kernel_named("cairn_wave_f8e5m2_nn_256x256"))  # fmt: skip
    assert named["name"] == "cairn_wave_f8e5m2_nn_256x256"
    assert choose(L.BF16, L.F32, 256, 256, 256, P + 2, P, P)["family"] == "generic"  # a off 16 bytes
    assert choose(L.BF16, L.F32, 256, 250, 256, P, P, P)["family"] == "generic"  # n % 4


def test_the_selector_refuses_what_no_kernel_computes():
    def status(**kw):
        base = dict(ab_type=L.BF16, c_type=L.F32, m=64, n=64, k=64, a=P, b=P, c=P)
        base.update(kw)
        d = L.desc(base.pop("ab_type"), base.pop("c_type"), base.pop("m"), base.pop("n"), base.pop("k"),
                   base.pop("a"), base.pop("b"), base.pop("c"), **base)  # fmt: skip
        return L.load().cairn_gemm_select(C.byref(d), None)
    assert status() == L.OK
    assert status(c_type=L.I32) == L.E_TYPE  # int32 output is for int8 operands
    assert status(c_type=L.BF16, accumulate=True) == L.E_TYPE  # accumulate adds into f32
    assert status(ab_type=L.I8, c_type=L.I32, act=L.ACT_RELU) == L.E_TYPE  # the accumulator itself, no epilogue
    assert status(lda=63) == L.E_SHAPE  # a row of 64 needs lda >= 64
    assert status(kernel=9999) == L.E_KERNEL
    assert status(k=60, kernel=L.kernel_named("cairn_wave_bf16_nn_256x256")) == L.E_KERNEL  # k % 8
    assert status(c=None) == L.E_ARG
    assert status(act=7) == L.E_ARG
    bad = L.desc(L.BF16, L.F32, 64, 64, 64, P, P, P)
    bad.version = 3  # no such version
    assert L.load().cairn_gemm_select(C.byref(bad), None) == L.E_ARG
    assert status(m=0, c=None) == L.OK  # nothing to do needs no pointers


def test_the_kernel_table_is_consistent():
    ks = L.kernels()
    assert len({k["name"] for k in ks}) == len(ks)
    for k in ks:
        assert k["lds_bytes"] <= 160 * 1024, k
        assert k["family"] in ("mfma", "wave", "generic", "skinny")
        if k["family"] == "wave":
            assert k["threads"] == 256 and k["tile_k"] in (32, 64)


# ------------------------------------------------------------------ the product never leans on the oracle


def test_the_product_does_not_reach_the_oracle():
    for path in [*(ROOT / "cairn_amd").rglob("*.py"), *(ROOT / "cairn_amd").rglob("*.hip"),
                 *(ROOT / "cairn_amd").rglob("*.cpp"), *(ROOT / "cairn_amd").rglob("*.hpp"), *(ROOT / "include").rglob("*.h*")]:  # fmt: skip
        text = path.read_text()
        assert "liboracle" not in text and "oracle_" not in text and "libcairnref" not in text, path


def test_a_missing_library_fails_loudly(tmp_path):
    code = f"""
import sys; sys.path.insert(0, {str(ROOT)!r})
from cairn_amd import lib as L
from pathlib import Path
L.LIBRARY = Path({str(tmp_path / 'absent.so')!r})
try:
    L.load()
except L.LibraryMissing as e:
    print("missing:", e)
"""
    done = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert "missing:" in done.stdout, done.stdout + done.stderr


def test_the_selector_splits_a_nearly_idle_last_round_where_a_workspace_is_given():
    """264 tiles of k = 8192 (one round and one tile an XCD): with the workspace cairn_gemm_workspace asks for, the
    last round's 8 tiles are shared along k by 4 units an XCD (no unit below 8 stages) and the tiling keeps the
    machine >= 97% busy; without a workspace it runs whole. C3's rounds (5.375 and 2.69: a quarter or more of the CUs
    busy in the last one) and C2 (one whole round) are not split by the selector: measured, a split round there was
    slower than the whole one (the clock rises when CUs idle)."""
    P = 1 << 20
    plain = L.desc(L.BF16, L.BF16, 2048, 8448, 8192, P, P, P)
    assert L.select(plain)["split_tiles"] == 0 and L.select(plain)["efficiency"] < 0.6
    need = L.workspace(plain)
    assert need == 2 * 8 * 32 * 256 * 256 * 4  # two partial tiles a unit, 32 units an XCD (256 stages / 8)
    given = L.desc(L.BF16, L.BF16, 2048, 8448, 8192, P, P, P, workspace=P, workspace_bytes=need)
    ch = L.select(given)
    assert ch["split_tiles"] == 8 and ch["split_units"] == 256 and ch["efficiency"] >= 0.97, ch
    for m, n, k, ta in ((8192, 11008, 4096, False), (4096, 11008, 8192, True), (4096, 4096, 4096, False)):
        d = L.desc(L.BF16, L.BF16, m, n, k, P, P, P, trans_a=ta, workspace=P, workspace_bytes=1 << 30)
        assert L.workspace(d) == 0 and L.select(d)["split_tiles"] == 0, (m, n, k)
    # Asked for explicitly, the MLP forward's last round splits over 256 units.
    fwd = L.desc(L.BF16, L.BF16, 8192, 11008, 4096, P, P, P, workspace=P, workspace_bytes=1 << 30, split_units=256)
    ch = L.select(fwd)
    assert ch["split_tiles"] == 96 and ch["split_units"] == 256 and ch["efficiency"] >= 0.97, ch


def test_an_explicit_split_is_checked_against_its_workspace():
    P = 1 << 20
    lib = L.load()

    def status(**kw):
        d = L.desc(L.BF16, L.BF16, 2048, 8448, 1024, P, P, P, **kw)
        return lib.cairn_gemm_select(C.byref(d), None)

    assert status(split_units=64) == L.E_SCRATCH  # no workspace at all
    assert status(split_units=64, workspace=P, workspace_bytes=64 * 2 * 256 * 1024) == L.OK
    assert status(split_units=64, workspace=P, workspace_bytes=64 * 2 * 256 * 1024 - 1) == L.E_SCRATCH
    # 272 tiles: 8 XCD blocks of 34, each splitting 2; one unit an XCD would span both tiles and more.
    d = L.desc(L.BF16, L.BF16, 2048, 8704, 1024, P, P, P, workspace=P, workspace_bytes=1 << 30, split_units=8)
    assert lib.cairn_gemm_select(C.byref(d), None) == L.E_ARG
    assert status(split_units=-2) == L.E_ARG
    assert status(workspace=P + 16, workspace_bytes=1 << 30) == L.E_ARG  # off 256 bytes
    # A version 1 descriptor (up to `kernel`) is read as such and never splits.
    old = L.desc(L.BF16, L.BF16, 8192, 11008, 4096, P, P, P, workspace=P, workspace_bytes=1 << 30)
    old.version = 1
    choice = L.Choice()
    assert lib.cairn_gemm_select(C.byref(old), C.byref(choice)) == L.OK and choice.split_tiles == 0


def test_the_bindings_use_the_headers_descriptor_versions():
    text = HEADER.read_text()
    assert int(re.search(r"#define CAIRN_GEMM_DESC_VERSION (\d+)u", text).group(1)) == L.DESC_VERSION
    assert int(re.search(r"#define CAIRN_QUANTIZE_DESC_VERSION (\d+)u", text).group(1)) == L.QUANTIZE_DESC_VERSION


def test_the_quantize_kernel_query_names_the_launch_form():
    """cairn_quantize_kernel, no GPU call: the fast kernel for whole aligned 8-element chunks, the general one
    otherwise; 4 rows a workgroup up to 4096 elements a row, 1 beyond; nothing for m = 0 or a refused descriptor."""
    X, Q, S = 1 << 20, 1 << 21, 1 << 22  # addresses only: nothing is read
    assert L.quantize_kernel(L.quantize_desc(L.BF16, L.I8, 8192, 4096, X, Q, S)) == "quantize_fast<bf16, i8, 4>"
    assert L.quantize_kernel(L.quantize_desc(L.F32, L.F8E4M3, 8, 4096, X, Q, S)) == "quantize_fast<f32, f8e4m3, 4>"
    assert L.quantize_kernel(L.quantize_desc(L.F32, L.F8E4M3, 8, 4104, X, Q, S)) == "quantize_fast<f32, f8e4m3, 1>"
    assert L.quantize_kernel(L.quantize_desc(L.F16, L.F8E5M2, 8, 8200, X, Q, S)) == "quantize_fast<f16, f8e5m2, 1>"
    assert L.quantize_kernel(L.quantize_desc(L.BF16, L.I8, 8, 4096, X + 2, Q, S)) == "quantize_rows<bf16, i8, 4>"
    assert L.quantize_kernel(L.quantize_desc(L.BF16, L.I8, 8, 4092, X, Q, S)) == "quantize_rows<bf16, i8, 4>"
    assert L.quantize_kernel(L.quantize_desc(L.BF16, L.I8, 8, 4096, X, Q, S, ldx=4100)) == "quantize_rows<bf16, i8, 4>"
    assert L.quantize_kernel(L.quantize_desc(L.BF16, L.I8, 0, 4096, X, Q, S)) is None
    assert L.quantize_kernel(L.quantize_desc(L.BF16, L.F16, 8, 4096, X, Q, S)) is None
    assert L.quantize_kernel(L.quantize_desc(L.BF16, L.I8, 8, 4096, X, Q, None)) is None


def test_the_selector_ranks_the_ring_kernel_first_then_the_mfma_kernel():
    """One kernel a family for a type and layout: the 256 x 256 ring kernel wherever its loads fit (measured faster at
    every bf16 shape of `bench.py --only selector`), the 128 x 128 MFMA kernel where only its chunks fit, else generic;
    and int8 at k <= 1024 with at most 256 MFMA tiles, where the MFMA kernel measured faster, on it."""
    for ab, tag in ((L.BF16, "bf16"), (L.F16, "f16"), (L.I8, "i8")):
        out = L.I32 if ab == L.I8 else L.BF16
        for m, n, k in ((4096, 4096, 4096), (256, 256, 4096), (300, 512, 2048), (8192, 11008, 4096), (4096, 4096, 1024)):
            assert L.select(L.desc(ab, out, m, n, k, P, P, P))["name"] == f"cairn_wave_{tag}_nn_256x256", (tag, m, n, k)
        # n = 128: b's k rows (NN, N-major) are closer than a 256-wide tile, too close for the ring's immediate offsets
        assert L.select(L.desc(ab, out, 4096, 128, 4096, P, P, P))["name"] == f"cairn_mfma_{tag}_nn_128x128"
        # n = 4: no 16-byte chunk of b's rows; only the generic kernel
        assert L.select(L.desc(ab, out, 4096, 4, 4096, P, P, P))["name"] == "cairn_generic_64x64"
    # int8 n = 520: the ring's N-major rows go in 16-byte chunks (16 columns), the MFMA kernel's in 8-byte ones
    assert L.select(L.desc(L.I8, L.I32, 300, 520, 2048, P, P, P))["name"] == "cairn_mfma_i8_nn_128x128"
    # int8, k <= 1024, at most 256 tiles of 128 x 128: the MFMA kernel; one tile more, or a longer k: the ring kernel
    for m, n, k, name in ((2048, 2048, 1024, "mfma"), (256, 4096, 1024, "mfma"), (300, 512, 64, "mfma"),
                          (2048, 2176, 1024, "wave"), (2048, 2048, 1040, "wave")):
        assert L.select(L.desc(L.I8, L.I32, m, n, k, P, P, P))["name"] == f"cairn_{name}_i8_nn_" + (
            "128x128" if name == "mfma" else "256x256"), (m, n, k)
    assert L.select(L.desc(L.BF16, L.BF16, 2048, 2048, 1024, P, P, P))["name"] == "cairn_wave_bf16_nn_256x256"
