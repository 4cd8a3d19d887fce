// The one-wave-a-SIMD GEMM (wave.hpp) for bf16 operands: the instances wave_bf16.inc lists.
#include "wave.hpp"

#include "wave_bf16.inc"
