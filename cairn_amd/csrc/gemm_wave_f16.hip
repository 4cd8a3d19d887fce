// The one-wave-a-SIMD GEMM (wave.hpp) for f16 operands: the instances wave_f16.inc lists.
#include "wave.hpp"

#include "wave_f16.inc"
