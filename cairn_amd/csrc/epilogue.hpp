// The fused epilogue of a wave's blocks of MFMA accumulators, applied block column by block column: the scales and
// bias a lane needs are loaded once per 32-column block, each output goes through the steps of `epilogue`
// (kernels.hpp) in their order and with their roundings, and the conversions to 16-bit outputs are packed.
//
// A wave holds FM x FN blocks of 32 x 32; in block (i, j), register 4 q + e of lane l is row 32 i + (l % 32), column
// 32 j + 8 q + 4 (l / 32) + e of the wave's part of c (tile.hpp, acc_m and acc_n). Absent terms are exact identities
// (a scale of 1, a bias of -0, which leaves every value, a zero's sign included, as it is), so one code path serves
// every combination without changing a bit of what the separate steps give.
#pragma once
#include <hip/hip_runtime.h>
#include <type_traits>
#include "kernels.hpp"
#include "mfma.hpp"
#include "tile.hpp"

namespace cairn::gemm {

// The row scale of each of the lane's rows r0 + 32 i + lane % 32 (1 where there is none or the row is past m).
template<int FM>
__device__ __forceinline__ void row_scales(const Params& p, int r0, int lane, float (&rs)[FM]) {
#pragma unroll
  for(int i = 0; i < FM; ++i) {
    const int m = r0 + 32 * i + (lane & 31);
    rs[i] = p.row_scale && m < p.m ? p.row_scale[m] : 1.0f;
  }
}

// The column scales and biases of the lane's 16 columns of a block column starting at n0: quad q, element e is
// column n0 + 8 q + 4 (lane / 32) + e (1 and -0 where there is none or the column is past n).
__device__ __forceinline__ void col_terms(const Params& p, int n0, int lane, float (&cs)[4][4], float (&bs)[4][4]) {
  const bool bias16 = p.bias_type == CAIRN_TYPE_BF16;
#pragma unroll
  for(int q = 0; q < 4; ++q) {
    const int n = n0 + 8 * q + 4 * (lane >> 5);
    const bool in = n < p.n;  // n and p.n are multiples of 4: the four columns are in or out together
#pragma unroll
    for(int e = 0; e < 4; ++e) {
      cs[q][e] = p.col_scale && in ? p.col_scale[n + e] : 1.0f;
      if(p.bias && in)
        bs[q][e] = bias16 ? widen_bf16(static_cast<const std::uint16_t*>(p.bias)[n + e])
                          : static_cast<const float*>(p.bias)[n + e];
      else bs[q][e] = -0.0f;
    }
  }
}

// The epilogue's form for one launch: its activation (ACT_SCALES: scales and nothing else, the W8A8 dequant, so the
// bias step, an add of -0 that changes no value, is left out) and whether a row or column scale is present (without
// one, the two multiplies by 1, which change no value either, are left out). Template arguments: callers branch on
// the form once, outside their loops, so that a loop holds only its own form's code (256 unrolled copies of GELU that
// a plain store jumps over still crowd the instruction cache).
constexpr int ACT_SCALES = -1;
template<int ACT, bool SCALED> struct Form {
  static constexpr int act = ACT;
  static constexpr bool scaled = SCALED;
};

// The epilogue's steps on one accumulator value, each an f32 rounding, in the order cairn_gemm.h states.
template<class F>
__device__ __forceinline__ float apply(float v, float rs, float cs, float bs) {
  if constexpr(F::scaled) {
    v = v * rs;
    v = v * cs;
  }
  if constexpr(F::act != ACT_SCALES) v = v + bs;
  if constexpr(F::act == CAIRN_ACT_RELU) v = v < 0.0f ? 0.0f : v;
  else if constexpr(F::act == CAIRN_ACT_GELU) v = gelu(v);
  return v;
}

// f(Form<...>{}) for the activation p.act names (ACT_SCALES where there is neither activation nor bias). GELU without
// scales (the MLP forward's bias + GELU) has a form of its own; the other forms keep the multiplies, whose cost is
// small beside their code: each form is another unrolled copy of the epilogue in every kernel, and more copies crowd
// the registers the main loop needs.
template<class G> __device__ __forceinline__ void with_form(const Params& p, G&& f) {
  if(p.act == CAIRN_ACT_GELU) {
    if(p.row_scale || p.col_scale) f(Form<CAIRN_ACT_GELU, true>{});
    else f(Form<CAIRN_ACT_GELU, false>{});
  } else if(p.act == CAIRN_ACT_RELU) {
    f(Form<CAIRN_ACT_RELU, true>{});
  } else if(!p.bias) {
    f(Form<ACT_SCALES, true>{});
  } else {
    f(Form<CAIRN_ACT_NONE, true>{});
  }
}

// RAW: the int32 accumulator itself is the output (int8 operands, c of int32, no epilogue); the kernel is built once
// each way, so that the two paths do not share (and hoist) the reads of the accumulators.
template<bool RAW, int FM, int FN, class Acc>
__device__ __forceinline__ void finish(const Params& p, const Acc (&acc)[FM][FN], int r0, int c0, int lane) {
  char* c = static_cast<char*>(p.c);
  const bool whole = r0 + 32 * FM <= p.m && c0 + 32 * FN <= p.n;
  const int row = lane & 31, half = lane >> 5;
  if constexpr(RAW) {
    {
#pragma unroll
      for(int i = 0; i < FM; ++i)
#pragma unroll
        for(int j = 0; j < FN; ++j)
#pragma unroll
          for(int q = 0; q < 4; ++q) {
            const int m = r0 + 32 * i + row, n = c0 + 32 * j + 8 * q + 4 * half;
            if(!whole && !(m < p.m && n < p.n)) continue;
            i32x4 w;
#pragma unroll
            for(int e = 0; e < 4; ++e) w[e] = int(acc[i][j][4 * q + e]);
            *reinterpret_cast<i32x4*>(c + (std::int64_t(m) * p.ldc + n) * 4) = w;
          }
      return;
    }
  } else {
  with_form(p, [&](auto form) {
  using F = decltype(form);
  float rs[FM];
  row_scales<FM>(p, r0, lane, rs);
#pragma unroll
  for(int j = 0; j < FN; ++j) {
    float cs[4][4], bs[4][4];
    col_terms(p, c0 + 32 * j, lane, cs, bs);
#pragma unroll
    for(int i = 0; i < FM; ++i)
#pragma unroll
      for(int q = 0; q < 4; ++q) {
        const int m = r0 + 32 * i + row, n = c0 + 32 * j + 8 * q + 4 * half;
        if(!whole && !(m < p.m && n < p.n)) continue;
        float v[4];
#pragma unroll
        for(int e = 0; e < 4; ++e) v[e] = apply<F>(float(acc[i][j][4 * q + e]), rs[i], cs[q][e], bs[q][e]);
        const std::int64_t at = std::int64_t(m) * p.ldc + n;
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
        } else if(p.c_type == CAIRN_TYPE_BF16) {
          u32x2 w;
          w[0] = narrow2_bf16(v[0], v[1]);
          w[1] = narrow2_bf16(v[2], v[3]);
          *reinterpret_cast<u32x2*>(c + at * 2) = w;
        } else {
          u32x2 w;
          w[0] = std::uint32_t(narrow_f16(v[0])) | (std::uint32_t(narrow_f16(v[1])) << 16);
          w[1] = std::uint32_t(narrow_f16(v[2])) | (std::uint32_t(narrow_f16(v[3])) << 16);
          *reinterpret_cast<u32x2*>(c + at * 2) = w;
        }
      }
  }
  });
  }
}

}  // namespace cairn::gemm
