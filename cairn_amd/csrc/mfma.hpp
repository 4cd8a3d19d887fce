// The matrix-core instructions the tiled kernels run, as one step each: D = P Q + C with P the first operand (its
// rows index the accumulator's rows) and Q the second. bf16 and f16 on v_mfma_f32_32x32x16_*, int8 on
// v_mfma_i32_32x32x32_i8; each operand register quad holds 16 bytes of k for one row of its matrix.
#pragma once
#include <hip/hip_runtime.h>
#include "kernels.hpp"
#include "tile.hpp"

namespace cairn::gemm {
using cairn::tile::u32x4;
using cairn::tile::u32x2;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));

template<int OP> struct Mfma;
template<> struct Mfma<OP_BF16> {
  using Acc = f32x16;
  static constexpr int ES = 2;
  __device__ static Acc step(u32x4 x, u32x4 y, Acc c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, x), __builtin_bit_cast(bf16x8, y), c,
                                                   0, 0, 0);
  }
};
template<> struct Mfma<OP_F16> {
  using Acc = f32x16;
  static constexpr int ES = 2;
  __device__ static Acc step(u32x4 x, u32x4 y, Acc c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, x), __builtin_bit_cast(f16x8, y), c, 0,
                                                  0, 0);
  }
};
template<> struct Mfma<OP_I8> {
  using Acc = i32x16;
  static constexpr int ES = 1;
  __device__ static Acc step(u32x4 x, u32x4 y, Acc c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4, x), __builtin_bit_cast(i32x4, y), c, 0, 0,
                                                 0);
  }
};

// The 8-bit floats on v_mfma_f32_32x32x64_f8f6f4 (OCP E4M3 or E5M2 for both operands; the scaled builtin with zero
// scale operands, which is the unscaled instruction): one step covers 64 bytes of k, each operand the two 16-byte
// k-steps of the int8 layout side by side. The instruction pairs the operands' bytes position by position, so any
// one order of k that both operands share gives the same sum.
typedef int i32x8 __attribute__((ext_vector_type(8)));
template<int FMT> struct Mfma8 {
  using Acc = f32x16;
  static constexpr int ES = 1;
  __device__ static Acc step(u32x4 x0, u32x4 x1, u32x4 y0, u32x4 y1, Acc c) {
    const i32x8 x = {int(x0[0]), int(x0[1]), int(x0[2]), int(x0[3]), int(x1[0]), int(x1[1]), int(x1[2]), int(x1[3])};
    const i32x8 y = {int(y0[0]), int(y0[1]), int(y0[2]), int(y0[3]), int(y1[0]), int(y1[1]), int(y1[2]), int(y1[3])};
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(x, y, c, FMT, FMT, 0, 0, 0, 0);
  }
};
template<> struct Mfma<OP_F8E4M3> : Mfma8<0> {};
template<> struct Mfma<OP_F8E5M2> : Mfma8<1> {};

// Quad q of one 32 x 32 accumulator block is row m, columns n .. n+3 (tile.hpp, acc_m / acc_n): the epilogue of
// those four outputs and their store, 16 bytes (f32, int32) or 8 (bf16, f16). The caller has checked m < p.m and
// n < p.n; n is a multiple of 4 and p.n too, so all four columns exist.
template<class Acc> __device__ inline void store_quad(const Params& p, int m, int n, const Acc& acc, int q) {
  char* c = static_cast<char*>(p.c);
  const std::int64_t at = std::int64_t(m) * p.ldc + n;
  if constexpr(sizeof(acc[0]) == 4 && !__is_same(decltype(+acc[0]), float)) {
    if(p.c_type == CAIRN_TYPE_I32) {
      i32x4 w;
#pragma unroll
      for(int e = 0; e < 4; ++e) w[e] = int(acc[4 * q + e]);
      *reinterpret_cast<i32x4*>(c + at * 4) = w;
      return;
    }
  }
  float v[4];
#pragma unroll
  for(int e = 0; e < 4; ++e) v[e] = float(acc[4 * q + e]);
  epilogue<4>(p, m, n, v);
  if(p.c_type == CAIRN_TYPE_F32) {
    float* out = reinterpret_cast<float*>(c + at * 4);
    if(p.accumulate) {
      const float4 old = *reinterpret_cast<const float4*>(out);
      v[0] = old.x + v[0];
      v[1] = old.y + v[1];
      v[2] = old.z + v[2];
      v[3] = old.w + v[3];
    }
    *reinterpret_cast<float4*>(out) = float4{v[0], v[1], v[2], v[3]};
  } else {
    std::uint16_t h[4];
#pragma unroll
    for(int e = 0; e < 4; ++e) h[e] = p.c_type == CAIRN_TYPE_BF16 ? narrow_bf16(v[e]) : narrow_f16(v[e]);
    u32x2 w;
    w[0] = std::uint32_t(h[0]) | (std::uint32_t(h[1]) << 16);
    w[1] = std::uint32_t(h[2]) | (std::uint32_t(h[3]) << 16);
    *reinterpret_cast<u32x2*>(c + at * 2) = w;
  }
}

}  // namespace cairn::gemm
