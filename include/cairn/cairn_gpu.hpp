// The header CAIRN-emitted device code includes by this name (src/cairn/compiler/device/tensor.py:75-76,
// lower/codegen.py:86,502). It chooses the machine device work runs on and brings what emitted code calls on it:
//
//   - HIP for gfx950 (cairn_hip.hpp; under hipcc also its device code, cairn_hip_kernels.hpp), so that
//     cr::tensor::launch<A>(cr::gpu::here(), ...) queues the gfx950 kernels of libcairn_gemm_gfx950.so;
//   - or, built with -DCAIRN_EMULATE by the host compiler, the host (cairn_emulate.hpp): the same program with its
//     device work run on the calling thread (`cairn build --emulate`, src/cairn/projects/toolchain.py:175-180).
//
// Then the thread's context and its scopes (cairn_here.hpp) and the operations on it (cairn_ops.hpp).
#pragma once
#include "cairn_runtime.hpp"
#if defined(CAIRN_EMULATE)
#include "cairn_emulate.hpp"
#else
#include "cairn_hip.hpp"
#if defined(__HIPCC__)
#include "cairn_hip_kernels.hpp"
#endif
#endif
#include "cairn_here.hpp"
#include "cairn_ops.hpp"
