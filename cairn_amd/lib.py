"""ctypes bindings of libcairn_gemm_gfx950.so, the library include/cairn_gemm.h declares.

The library is the product: there is no fallback. If it has not been built (python -m cairn_amd.build), loading
raises LibraryMissing, and every entry that would run on the GPU fails with it.
"""

from __future__ import annotations

import ctypes as C
from pathlib import Path

from cairn_amd import identity

HERE = Path(__file__).resolve().parent
LIBRARY = HERE / "libcairn_gemm_gfx950.so"

# enum cairn_type, cairn_act, cairn_status
F32, F16, BF16, F8E4M3, F8E5M2, I8, I32 = range(7)
ACT_NONE, ACT_RELU, ACT_GELU = range(3)
OK, E_SHAPE, E_TYPE, E_KERNEL, E_ARG, E_HIP, E_SCRATCH = range(7)
DESC_VERSION = 2
# enum cairn_scale_mode, cairn_quant_status
SCALE_ROW_ABSMAX, SCALE_ROW, SCALE_TENSOR = range(3)
QUANT_BAD_SCALE, QUANT_NAN = 1, 2
QUANTIZE_DESC_VERSION = 1
STATIC_SCRATCH = 64 << 20  # CAIRN_GEMM_STATIC_SCRATCH
FAMILY = {0: "mfma", 1: "generic", 2: "skinny", 4: "wave"}
TYPE_NAMES = {F32: "f32", F16: "f16", BF16: "bf16", F8E4M3: "f8e4m3", F8E5M2: "f8e5m2", I8: "i8", I32: "i32"}


class LibraryMissing(RuntimeError):
    pass


class GemmError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"cairn_gemm: {message} (status {status})")
        self.status = status


class Desc(C.Structure):
    """struct cairn_gemm_desc."""

    _fields_ = [
        ("version", C.c_uint32),
        ("ab_type", C.c_int32),
        ("c_type", C.c_int32),
        ("trans_a", C.c_int32),
        ("trans_b", C.c_int32),
        ("m", C.c_uint64),
        ("n", C.c_uint64),
        ("k", C.c_uint64),
        ("lda", C.c_uint64),
        ("ldb", C.c_uint64),
        ("ldc", C.c_uint64),
        ("a", C.c_void_p),
        ("b", C.c_void_p),
        ("c", C.c_void_p),
        ("accumulate", C.c_int32),
        ("act", C.c_int32),
        ("bias", C.c_void_p),
        ("bias_type", C.c_int32),
        ("row_scale", C.c_void_p),
        ("col_scale", C.c_void_p),
        ("kernel", C.c_int32),
        ("workspace", C.c_void_p),
        ("workspace_bytes", C.c_uint64),
        ("split_units", C.c_int32),
    ]


class QuantizeDesc(C.Structure):
    """struct cairn_quantize_desc."""

    _fields_ = [
        ("version", C.c_uint32),
        ("x_type", C.c_int32),
        ("q_type", C.c_int32),
        ("mode", C.c_int32),
        ("m", C.c_uint64),
        ("k", C.c_uint64),
        ("ldx", C.c_uint64),
        ("ldq", C.c_uint64),
        ("x", C.c_void_p),
        ("q", C.c_void_p),
        ("scale", C.c_void_p),
        ("status", C.c_void_p),
    ]


class Kernel(C.Structure):
    """struct cairn_gemm_kernel."""

    _fields_ = [
        ("id", C.c_int32),
        ("ab_type", C.c_int32),
        ("trans_a", C.c_int32),
        ("trans_b", C.c_int32),
        ("tile_m", C.c_int32),
        ("tile_n", C.c_int32),
        ("tile_k", C.c_int32),
        ("threads", C.c_int32),
        ("lds_bytes", C.c_int32),
        ("family", C.c_int32),
        ("name", C.c_char * 48),
    ]


class Choice(C.Structure):
    """struct cairn_gemm_choice."""

    _fields_ = [
        ("kernel", C.c_int32),
        ("family", C.c_int32),
        ("tile_m", C.c_int32),
        ("tile_n", C.c_int32),
        ("tile_k", C.c_int32),
        ("workgroups", C.c_uint64),
        ("waves", C.c_double),
        ("efficiency", C.c_double),
        ("split_tiles", C.c_int32),
        ("split_units", C.c_int32),
        ("split_bytes", C.c_uint64),
    ]


# Every symbol include/cairn_gemm.h declares, with its ctypes signature.
SZ = C.c_size_t
_MMA = [SZ, SZ, SZ, SZ, C.c_void_p, SZ, C.c_void_p, SZ, C.c_void_p]
SIGNATURES = {
    "cairn_gemm_run": (C.c_int, [C.POINTER(Desc), C.c_void_p]),
    "cairn_gemm_run_static": (C.c_int, [C.POINTER(Desc), C.c_void_p]),
    "cairn_gemm_select": (C.c_int, [C.POINTER(Desc), C.POINTER(Choice)]),
    "cairn_gemm_workspace": (C.c_int, [C.POINTER(Desc), C.POINTER(C.c_uint64)]),
    "cairn_gemm_kernel_count": (C.c_int, []),
    "cairn_gemm_kernel_info": (C.c_int, [C.c_int32, C.POINTER(Kernel)]),
    "cairn_gemm_status_string": (C.c_char_p, [C.c_int]),
    "cairn_gemm_mma": (C.c_int, [C.c_int32, SZ, SZ, SZ, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p]),
    "cairn_gemm_device_stream": (None, [C.c_void_p]),
    "cairn_quantize_run": (C.c_int, [C.POINTER(QuantizeDesc), C.c_void_p]),
    "cairn_quantize_kernel": (C.c_char_p, [C.POINTER(QuantizeDesc)]),
    **{f"cf_mma_{f}": (None, _MMA) for f in ("f32", "f16", "bf16", "f8e4m3", "f8e5m2")},
    **{f"cf_mma_{f}_device": (None, _MMA) for f in ("f16", "bf16", "f8e4m3", "f8e5m2")},
    **{f"cq_mma_{f}_device": (None, [C.c_void_p, *_MMA]) for f in ("f16", "bf16", "f8e4m3", "f8e5m2")},
}
DATA_SYMBOLS = [identity.declared()]  # the interface identity include/cairn_gemm.h names

_lib: C.CDLL | None = None


def load() -> C.CDLL:
    """The library, loaded once, every declared entry typed. Raises LibraryMissing if it is not built."""
    global _lib
    if _lib is None:
        if not LIBRARY.exists():
            raise LibraryMissing(f"{LIBRARY} is not built: run `python -m cairn_amd.build` (hipcc, gfx950)")
        lib = C.CDLL(str(LIBRARY))
        for name, (res, args) in SIGNATURES.items():
            f = getattr(lib, name)
            f.restype = res
            f.argtypes = args
        _lib = lib
    return _lib


def status_string(status: int) -> str:
    return load().cairn_gemm_status_string(status).decode()


def desc(ab_type: int, c_type: int, m: int, n: int, k: int, a=None, b=None, c=None, *, trans_a: bool = False,
         trans_b: bool = False, lda: int = 0, ldb: int = 0, ldc: int = 0, accumulate: bool = False,
         act: int = ACT_NONE, bias=None, bias_type: int = F32, row_scale=None, col_scale=None,
         kernel: int = 0, workspace=None, workspace_bytes: int = 0, split_units: int = 0) -> Desc:  # fmt: skip
    """A cairn_gemm_desc; pointers are ints (device addresses) or None."""
    return Desc(DESC_VERSION, ab_type, c_type, int(trans_a), int(trans_b), m, n, k, lda, ldb, ldc, a, b, c,
                int(accumulate), act, bias, bias_type, row_scale, col_scale, kernel, workspace, workspace_bytes,
                split_units)  # fmt: skip


def workspace(d: Desc) -> int:
    """The bytes a split last round of `d` would use (cairn_gemm_workspace)."""
    out = C.c_uint64(0)
    s = load().cairn_gemm_workspace(C.byref(d), C.byref(out))
    if s != OK:
        raise GemmError(s, status_string(s))
    return out.value


def run(d: Desc, stream: int | None = None) -> None:
    s = load().cairn_gemm_run(C.byref(d), stream)
    if s != OK:
        raise GemmError(s, status_string(s))


def quantize_desc(x_type: int, q_type: int, m: int, k: int, x=None, q=None, scale=None, *,
                  mode: int = SCALE_ROW_ABSMAX, ldx: int = 0, ldq: int = 0, status=None) -> QuantizeDesc:  # fmt: skip
    """A cairn_quantize_desc; pointers are ints (device addresses) or None."""
    return QuantizeDesc(QUANTIZE_DESC_VERSION, x_type, q_type, mode, m, k, ldx, ldq, x, q, scale, status)


def quantize(d: QuantizeDesc, stream: int | None = None) -> None:
    s = load().cairn_quantize_run(C.byref(d), stream)
    if s != OK:
        raise GemmError(s, status_string(s))


def quantize_kernel(d: QuantizeDesc) -> str | None:
    """The name of the kernel cairn_quantize_run launches for `d` (None: refused, or nothing to launch)."""
    name = load().cairn_quantize_kernel(C.byref(d))
    return name.decode() if name else None


def select(d: Desc) -> dict:
    choice = Choice()
    s = load().cairn_gemm_select(C.byref(d), C.byref(choice))
    if s != OK:
        raise GemmError(s, status_string(s))
    info = kernel_info(choice.kernel)
    return {"kernel": choice.kernel, "name": info["name"], "family": FAMILY[choice.family], "tile_m": choice.tile_m,
            "tile_n": choice.tile_n, "tile_k": choice.tile_k, "workgroups": choice.workgroups,
            "waves": choice.waves, "efficiency": choice.efficiency, "split_tiles": choice.split_tiles,
            "split_units": choice.split_units, "split_bytes": choice.split_bytes}  # fmt: skip


def kernel_info(kid: int) -> dict:
    k = Kernel()
    s = load().cairn_gemm_kernel_info(kid, C.byref(k))
    if s != OK:
        raise GemmError(s, status_string(s))
    return {"id": k.id, "name": k.name.decode(), "ab_type": k.ab_type, "trans_a": bool(k.trans_a),
            "trans_b": bool(k.trans_b), "tile_m": k.tile_m, "tile_n": k.tile_n, "tile_k": k.tile_k,
            "threads": k.threads, "lds_bytes": k.lds_bytes, "family": FAMILY[k.family]}  # fmt: skip


def kernels() -> list[dict]:
    return [kernel_info(i) for i in range(1, load().cairn_gemm_kernel_count() + 1)]


def kernel_named(name: str) -> int:
    for k in kernels():
        if k["name"] == name:
            return k["id"]
    raise KeyError(name)
