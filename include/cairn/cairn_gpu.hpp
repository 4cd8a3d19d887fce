// The header CAIRN-emitted device code includes by this name (src/cairn/compiler/device/tensor.py:75-76,
// lower/codegen.py:86,502): with the gfx950 runtime on the include path it brings the HIP machine, so that
// cr::tensor::launch<A>(cr::gpu::here(), ...) queues the gfx950 kernels and cr::gpu::use_stream, Held and Enqueued
// keep their meaning (src/cairn/runtime/cairn_exec.hpp:25-67); under hipcc it also brings the device regions, owners,
// reductions, scans and queued work of cairn_hip_exec.hpp (cairn_exec.hpp:68-230).
#pragma once
#include "cairn_hip.hpp"
#include "cairn_runtime.hpp"
#if defined(__HIPCC__)
#include "cairn_hip_exec.hpp"
#endif
