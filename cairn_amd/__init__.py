"""cairn_amd: CAIRN's tensor-core GEMM runtime for the MI355X (gfx950).

The product is native: libcairn_gemm_gfx950.so (HIP kernels + C ABI, include/cairn_gemm.h) and the C++20 surface in
include/cairn/. This package is the Python toolchain around it: build (cairn_amd.build), ctypes bindings (cairn_amd.lib),
HIP plumbing for tests and benchmarks (cairn_amd.hip) and the perf model that reads the tile selector (cairn_amd.perf).
"""

__version__ = "0.1.0"
