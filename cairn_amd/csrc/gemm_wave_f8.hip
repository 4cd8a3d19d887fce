// The one-wave-a-SIMD GEMM (wave.hpp) for the 8-bit floats operands: the instances wave_f8.inc lists.
#include "wave.hpp"

#include "wave_f8.inc"
