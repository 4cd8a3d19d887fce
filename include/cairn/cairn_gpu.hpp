// The header CAIRN-emitted device code includes by this name (src/cairn/compiler/device/tensor.py:75-76,
// lower/codegen.py:86,502): with the gfx950 runtime on the include path it brings the HIP machine, so that
// cr::tensor::launch<A>(cr::gpu::here(), ...) queues the gfx950 kernels and cr::gpu::use_stream, Held and Enqueued
// keep their meaning (src/cairn/runtime/cairn_exec.hpp:25-67).
#pragma once
#include "cairn_hip.hpp"
#include "cairn_runtime.hpp"
