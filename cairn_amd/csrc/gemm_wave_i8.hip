// The one-wave-a-SIMD GEMM (wave.hpp) for i8 operands: the instances wave_i8.inc lists.
#include "wave.hpp"

#include "wave_i8.inc"
