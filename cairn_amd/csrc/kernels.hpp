// What every GEMM kernel of the library takes, and the epilogue they all share: the per-launch parameters, the
// output roundings and the fused bias / activation / dequant-scale step. Device code only; the host side of the
// library (capi.cpp) fills a Params from a cairn_gemm_desc.
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>
#include "../../include/cairn_gemm.h"
#include "tile.hpp"

namespace cairn::gemm {

// The matrix-core operations the tiled kernels run on.
enum Op { OP_BF16 = 0, OP_F16 = 1, OP_I8 = 2, OP_F8E4M3 = 3, OP_F8E5M2 = 4 };

// One launch. Matrices are the caller's: a is m x k (trans_a: stored k x m), b is k x n (trans_b: stored n x k), c
// is m x n; ld* count elements between stored rows. Extents fit int32 (the host checks).
struct Params {
  const void* a;
  const void* b;
  void* c;
  std::int64_t lda, ldb, ldc;
  int m, n, k;
  int tiles_m, tiles_n;  // the output tiles, for kernels that tile
  int group;             // tile rows walked together for L2 reuse
  int trans_a, trans_b;  // a stored k x m; b stored n x k
  int a_type;            // CAIRN_TYPE_* of both operands
  int c_type;            // CAIRN_TYPE_* of the output
  int accumulate;        // f32 output: c = c_old + result
  int act;               // CAIRN_ACT_*
  const void* bias;      // per column, or null
  int bias_type;         // CAIRN_TYPE_F32 or CAIRN_TYPE_BF16
  const float* row_scale;
  const float* col_scale;
  int rows16;            // every row of c starts on 16 bytes (c 16-byte aligned, ldc a multiple of 16 bytes)
  int whole_tiles;       // workgroups of the whole-tile pass (workgroup b: tile id whole_id(split, b))
  cairn::tile::Split split;  // the split last round (split.tiles 0: none)
  void* work;            // the split round's partial tiles: 2 split.units slots of BM x BN 32-bit values
};

__device__ inline std::uint32_t as_bits(float x) { return __builtin_bit_cast(std::uint32_t, x); }
__device__ inline float from_bits(std::uint32_t u) { return __builtin_bit_cast(float, u); }

// f32 -> bf16, round to nearest even; past the largest finite value infinity; a NaN becomes the quiet NaN 0x7fc0
// with its sign. These are the rules of the reference's narrow<bf16> (src/cairn/runtime/cairn_float.hpp:100-110),
// applied to an f32, which is exact as a double.
__device__ inline std::uint16_t narrow_bf16(float x) {
  const std::uint32_t u = as_bits(x);
  if((u & 0x7fffffffu) > 0x7f800000u) return std::uint16_t(((u >> 16) & 0x8000u) | 0x7fc0u);
  return std::uint16_t((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}
// Two f32 -> bf16 in one instruction (v_cvt_pk_bf16_f32: nearest even, subnormals kept as the kernels' f32 mode
// keeps them, overflow to infinity), x in the low half. Equal to narrow_bf16 on every finite value and every infinity;
// a NaN stays a NaN, its payload the instruction's (the multiply's contract promises no particular NaN).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
__device__ inline std::uint32_t narrow2_bf16(float x, float y) {
  const bf16x2_t v = {static_cast<__bf16>(x), static_cast<__bf16>(y)};
  return __builtin_bit_cast(std::uint32_t, v);
}
// f32 -> f16, round to nearest even (the conversion's mode), overflow to infinity.
__device__ inline std::uint16_t narrow_f16(float x) {
  const _Float16 h = static_cast<_Float16>(x);
  return __builtin_bit_cast(std::uint16_t, h);
}
__device__ inline float widen_bf16(std::uint16_t b) { return from_bits(std::uint32_t(b) << 16); }

// GELU in its erf form, x Phi(x) = 0.5 x (1 + erf(x / sqrt 2)), in f32 and without branches (the library erff takes
// two paths by |x|, and a wave whose lanes straddle them runs both). Phi(x) is 1 - h for x >= 0 and h otherwise, with
// h = Phi(-|x|) = erfc(z) / 2, z = |x| / sqrt 2, so nothing subtracts near-equal values. h is written
// t 2^(q(t) - z^2 log2 e) with t = 1 / (1 + P z): q(t) = log2(erfcx(z) (1 + P z)) - 1 is smooth on t in (0, 1], and
// its degree-8 polynomial below is this build's minimax fit (iteratively reweighted least squares against scipy's
// erfcx, P = 0.38, over |x| <= 13.2, each coefficient rounded to f32 before the lower ones were refitted): absolute
// error 9.4e-8, so h keeps a relative error of that size for every x
// (the form of Press, Teukolsky, Vetterling and Flannery, Numerical Recipes, 2nd ed., section 6.2, erfcc, with a
// shorter fit). Evaluated in f32 with fused steps, the hardware's reciprocal and 2^x (1 ulp each), and the
// exponent's -z^2 log2 e inside one fma: relative error at most 4.6e-7 for |x| <= 1, 1.9e-6 for |x| <= 6, 7.7e-6 out
// to |x| = 13, where GELU reaches f32's smallest normals (tests/test_gelu_form.py). 20 instructions a value, two of
// them the reciprocal and 2^x. +inf gives +inf; NaN, and -inf (0 * inf), give NaN, as the erff form does.
__device__ inline float gelu(float x) {
  const float t = __builtin_amdgcn_rcpf(__builtin_fmaf(__builtin_fabsf(x), 0.268700577f, 1.0f));  // P / sqrt 2
  float q = -0.35370594f;
  q = __builtin_fmaf(q, t, 1.7261575f);
  q = __builtin_fmaf(q, t, -3.1757226f);
  q = __builtin_fmaf(q, t, 2.7078722f);
  q = __builtin_fmaf(q, t, -1.4281899f);
  q = __builtin_fmaf(q, t, 0.77864224f);
  q = __builtin_fmaf(q, t, 0.5123964f);
  q = __builtin_fmaf(q, t, 1.4548278f);
  q = __builtin_fmaf(q, t, -3.2222776f);
  const float arg = __builtin_fmaf(-x, x * 0.721347520f, q);  // q - x^2 (log2 e) / 2
  const float h = t * __builtin_amdgcn_exp2f(arg);
  return x * (x >= 0.0f ? 1.0f - h : h);
}

// The epilogue of the outputs (m, n0 .. n0+count-1) of one row, on f32 values v: each step an f32 rounding, in this
// order: times row_scale[m], times col_scale[n], plus bias[n], the activation, then (f32 output with accumulate)
// plus the old value. A NaN passes ReLU as a NaN.
template<int COUNT> __device__ inline void epilogue(const Params& p, int m, int n0, float (&v)[COUNT]) {
  if(p.row_scale) {
    const float s = p.row_scale[m];
    for(int t = 0; t < COUNT; ++t) v[t] = v[t] * s;
  }
  if(p.col_scale)
    for(int t = 0; t < COUNT; ++t) v[t] = v[t] * p.col_scale[n0 + t];
  if(p.bias) {
    if(p.bias_type == CAIRN_TYPE_BF16) {
      const std::uint16_t* b = static_cast<const std::uint16_t*>(p.bias);
      for(int t = 0; t < COUNT; ++t) v[t] = v[t] + widen_bf16(b[n0 + t]);
    } else {
      const float* b = static_cast<const float*>(p.bias);
      for(int t = 0; t < COUNT; ++t) v[t] = v[t] + b[n0 + t];
    }
  }
  if(p.act == CAIRN_ACT_RELU)
    for(int t = 0; t < COUNT; ++t) v[t] = v[t] < 0.0f ? 0.0f : v[t];
  else if(p.act == CAIRN_ACT_GELU)
    for(int t = 0; t < COUNT; ++t) v[t] = gelu(v[t]);
}

}  // namespace cairn::gemm
