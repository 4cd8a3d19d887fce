// The generic GEMM: any m, n, k, layout, leading dimension and alignment, every storage float. It exists for the
// shapes the tiled kernel's 16-byte chunks cannot cover (k or a leading dimension off a multiple of 8, misaligned
// pointers, odd n) and for the 8-bit floats, which it widens to f16 exactly as the reference does
// (src/cairn/runtime/cairn_tensor.hpp:123-135: every f8e4m3 and f8e5m2 value is an f16). Correct first, not fast:
// 64 x 64 tiles, four waves each holding one 32 x 32 MFMA block, k in steps of one MFMA, every element loaded alone
// with its bounds checked, staged K-major in LDS.
#include <hip/hip_runtime.h>
#include "kernels.hpp"

namespace cairn::gemm {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef std::uint32_t w32x4 __attribute__((ext_vector_type(4)));

// An OCP E4M3 pattern as the f16 pattern of the same value: bias 7 to bias 15, subnormals normalized, the one NaN
// (exponent and fraction all ones) to f16's quiet NaN.
__device__ inline std::uint16_t e4m3_as_f16(std::uint8_t x) {
  const std::uint16_t sign = std::uint16_t((x & 0x80u) << 8);
  const unsigned e = (x >> 3) & 15u, f = x & 7u;
  if(e == 15u && f == 7u) return sign | 0x7e00u;
  if(e == 0u) {
    if(f == 0u) return sign;
    const int lead = f >= 4u ? 2 : (f >= 2u ? 1 : 0);  // f * 2^-9 = 1.xx * 2^(lead - 9)
    return std::uint16_t(sign | ((lead + 6) << 10) | ((f - (1u << lead)) << (10 - lead)));
  }
  return std::uint16_t(sign | ((e + 8u) << 10) | (f << 7));
}
// E5M2 is the top byte of the f16 of the same value.
__device__ inline std::uint16_t e5m2_as_f16(std::uint8_t x) { return std::uint16_t(x) << 8; }

// Element (r, q) of an operand whose stored matrix is row-major with `ld` between rows (trans: stored transposed),
// as the MFMA's 16-bit pattern (or int8 byte); zero outside rows x cols.
__device__ inline std::uint32_t element(const void* base, int type, bool trans, std::int64_t ld, int r, int q, int rows,
                                        int cols) {
  if(r >= rows || q >= cols) return 0;
  const std::int64_t at = trans ? std::int64_t(q) * ld + r : std::int64_t(r) * ld + q;
  switch(type) {
    case CAIRN_TYPE_F16:
    case CAIRN_TYPE_BF16: return static_cast<const std::uint16_t*>(base)[at];
    case CAIRN_TYPE_F8E4M3: return e4m3_as_f16(static_cast<const std::uint8_t*>(base)[at]);
    case CAIRN_TYPE_F8E5M2: return e5m2_as_f16(static_cast<const std::uint8_t*>(base)[at]);
    default: return static_cast<const std::uint8_t*>(base)[at];  // int8
  }
}

template<bool I8> __global__ void __launch_bounds__(256) generic_gemm(Params p) {
  constexpr int KS = I8 ? 32 : 16;  // k per MFMA: 32 bytes of every row
  __shared__ __attribute__((aligned(16))) std::uint8_t as[64][32], bs[64][32];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int row0 = int(blockIdx.x / unsigned(p.tiles_n)) * 64, col0 = int(blockIdx.x % unsigned(p.tiles_n)) * 64;
  const bool ta = p.trans_a, tb = p.trans_b;
  const int ctype = p.c_type;

  typename std::conditional<I8, i32x16, f32x16>::type acc{};
  for(int k0 = 0; k0 < p.k; k0 += KS) {
    for(int e = t; e < 64 * KS; e += 256) {
      const int r = e / KS, q = e % KS;
      const std::uint32_t x = element(p.a, p.a_type, ta, p.lda, row0 + r, k0 + q, p.m, p.k);
      const std::uint32_t y = element(p.b, p.a_type, !tb, p.ldb, col0 + r, k0 + q, p.n, p.k);
      if(I8) {
        as[r][q] = std::uint8_t(x);
        bs[r][q] = std::uint8_t(y);
      } else {
        reinterpret_cast<std::uint16_t*>(as[r])[q] = std::uint16_t(x);
        reinterpret_cast<std::uint16_t*>(bs[r])[q] = std::uint16_t(y);
      }
    }
    __syncthreads();
    // Lane l holds 16 bytes of row l%32 starting at byte 16 * (l / 32), in both operands.
    const w32x4 xa = *reinterpret_cast<const w32x4*>(&as[wm * 32 + (lane & 31)][16 * (lane >> 5)]);
    const w32x4 xb = *reinterpret_cast<const w32x4*>(&bs[wn * 32 + (lane & 31)][16 * (lane >> 5)]);
    if constexpr(I8) {
      acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4, xb), __builtin_bit_cast(i32x4, xa), acc,
                                                  0, 0, 0);
    } else if(p.a_type == CAIRN_TYPE_BF16) {
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, xb), __builtin_bit_cast(bf16x8, xa),
                                                    acc, 0, 0, 0);
    } else {
      acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, xb), __builtin_bit_cast(f16x8, xa), acc,
                                                   0, 0, 0);
    }
    __syncthreads();
  }
  // Register r of lane l: row l%32, column 8 (r/4) + 4 (l/32) + r%4 of the wave's block.
  const int m = row0 + wm * 32 + (lane & 31);
  if(m >= p.m) return;
#pragma unroll
  for(int r = 0; r < 16; ++r) {
    const int n = col0 + wn * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
    if(n >= p.n) continue;
    const std::int64_t at = std::int64_t(m) * p.ldc + n;
    if(I8 && ctype == CAIRN_TYPE_I32) {
      static_cast<int*>(p.c)[at] = int(acc[r]);
      continue;
    }
    float v[1] = {float(acc[r])};
    epilogue<1>(p, m, n, v);
    if(ctype == CAIRN_TYPE_F32) {
      float* out = static_cast<float*>(p.c) + at;
      *out = p.accumulate ? *out + v[0] : v[0];
    } else {
      static_cast<std::uint16_t*>(p.c)[at] = ctype == CAIRN_TYPE_BF16 ? narrow_bf16(v[0]) : narrow_f16(v[0]);
    }
  }
}

}  // namespace cairn::gemm

// 64 x 64 tiles.
hipError_t cairn_generic(const cairn::gemm::Params& p0, hipStream_t s) {
  cairn::gemm::Params p = p0;
  p.tiles_m = (p.m + 63) / 64;
  p.tiles_n = (p.n + 63) / 64;
  const dim3 grid(unsigned(p.tiles_m) * unsigned(p.tiles_n));
  if(p.a_type == CAIRN_TYPE_I8) hipLaunchKernelGGL(cairn::gemm::generic_gemm<true>, grid, dim3(256), 0, s, p);
  else hipLaunchKernelGGL(cairn::gemm::generic_gemm<false>, grid, dim3(256), 0, s, p);
  return hipGetLastError();
}
