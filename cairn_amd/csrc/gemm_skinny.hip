// The skinny GEMM: m <= 16 rows of a (a decode step's tokens) against b stored n x k, K-contiguous (a weight matrix
// as a linear layer keeps it), bf16 in, f32 accumulate. At m <= 16 the work is 2 m flops per b element, far below
// the ridge of the roofline, so the kernel is built around streaming b from HBM once: every b byte is read by
// exactly one 16-byte load, 8 columns' worth of loads in flight per lane, and the matrix cores do the arithmetic
// (v_mfma_f32_16x16x32_bf16, its 16 rows holding a's m rows and zeros) so the vector ALUs never bound it.
//
// A workgroup of SPLIT waves owns 16 * GROUPS columns; each wave walks its own contiguous share of k for all of
// them, and the waves' partial sums meet in LDS, added in wave order, so two runs give the same bits. The reference
// has no decode path: its one tiling runs a 1 x n x k call as 64 x 64 tiles (src/cairn/runtime/cairn_tensor.hpp:206-221).
#include <hip/hip_runtime.h>
#include "kernels.hpp"

namespace cairn::gemm {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef std::uint32_t w32x4 __attribute__((ext_vector_type(4)));

__device__ inline __amdgpu_buffer_rsrc_t span(const void* base, std::int64_t bytes) {
  const std::int64_t capped = bytes < 0 ? 0 : (bytes > 0x7fffffffLL ? 0x7fffffffLL : bytes);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)capped, 0x00020000);
}
constexpr int NOWHERE = 0x7fffffff;

template<int GROUPS, int SPLIT, int UNROLL> __global__ void __launch_bounds__(64 * SPLIT) skinny_gemm(Params p) {
  __shared__ f32x4 partial[SPLIT][GROUPS][64];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int n0 = int(blockIdx.x) * 16 * GROUPS;
  const int row = lane & 15, piece = lane >> 4;  // MFMA operand: row (of a, or column of b) and 8-element k piece

  // b's rows n0 .. n0 + 16 * GROUPS, from their first element; a whole.
  const char* bp = static_cast<const char*>(p.b) + std::int64_t(n0) * p.ldb * 2;
  const std::int64_t bbytes = (std::int64_t(p.n - 1) * p.ldb + p.k) * 2 - std::int64_t(n0) * p.ldb * 2;
  const __amdgpu_buffer_rsrc_t rb = span(bp, bbytes);
  const __amdgpu_buffer_rsrc_t ra = span(p.a, (std::int64_t(p.m - 1) * p.lda + p.k) * 2);
  int boff[GROUPS];
#pragma unroll
  for(int g = 0; g < GROUPS; ++g)
    boff[g] = n0 + 16 * g + row < p.n ? int((16 * g + row) * p.ldb * 2) + 16 * piece : NOWHERE;
  const int aoff = row < p.m ? int(row * p.lda * 2) + 16 * piece : NOWHERE;

  // This wave's k-steps of 32: [first, last).
  const int steps = (p.k + 31) / 32;
  const int first = int(std::int64_t(steps) * wave / SPLIT), last = int(std::int64_t(steps) * (wave + 1) / SPLIT);
  f32x4 acc[GROUPS];
#pragma unroll
  for(int g = 0; g < GROUPS; ++g) acc[g] = f32x4{0, 0, 0, 0};

  auto fetch = [&](int step, w32x4& xa, w32x4 (&xb)[GROUPS]) {
    const int k = step * 32 + 8 * piece;  // this lane's 8 elements of k
    const bool inside = step < last && k < p.k;
    xa = __builtin_bit_cast(w32x4, __builtin_amdgcn_raw_buffer_load_b128(ra, inside && aoff != NOWHERE ? aoff + step * 64 : NOWHERE, 0, 0));
#pragma unroll
    for(int g = 0; g < GROUPS; ++g)
      xb[g] = __builtin_bit_cast(
          w32x4, __builtin_amdgcn_raw_buffer_load_b128(rb, inside && boff[g] != NOWHERE ? boff[g] + step * 64 : NOWHERE, 0, 0));
  };
  for(int s = first; s < last; s += UNROLL) {
    w32x4 xa[UNROLL], xb[UNROLL][GROUPS];
#pragma unroll
    for(int u = 0; u < UNROLL; ++u) fetch(s + u, xa[u], xb[u]);
#pragma unroll
    for(int u = 0; u < UNROLL; ++u)
#pragma unroll
      for(int g = 0; g < GROUPS; ++g)
        acc[g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, xa[u]),
                                                         __builtin_bit_cast(bf16x8, xb[u][g]), acc[g], 0, 0, 0);
  }

#pragma unroll
  for(int g = 0; g < GROUPS; ++g) partial[wave][g][lane] = acc[g];
  __syncthreads();
  if(wave) return;
  // Lane l holds rows 4 (l/16) .. +3 of column n0 + 16 g + l%16.
#pragma unroll
  for(int g = 0; g < GROUPS; ++g) {
    f32x4 sum = partial[0][g][lane];
#pragma unroll
    for(int w = 1; w < SPLIT; ++w) sum = sum + partial[w][g][lane];
    const int n = n0 + 16 * g + (lane & 15);
    if(n >= p.n) continue;
#pragma unroll
    for(int r = 0; r < 4; ++r) {
      const int m = 4 * (lane >> 4) + r;
      if(m >= p.m) continue;
      float v[1] = {sum[r]};
      epilogue<1>(p, m, n, v);
      const std::int64_t at = std::int64_t(m) * p.ldc + n;
      if(p.c_type == CAIRN_TYPE_F32) {
        float* out = static_cast<float*>(p.c) + at;
        *out = p.accumulate ? *out + v[0] : v[0];
      } else {
        static_cast<std::uint16_t*>(p.c)[at] = p.c_type == CAIRN_TYPE_BF16 ? narrow_bf16(v[0]) : narrow_f16(v[0]);
      }
    }
  }
}

}  // namespace cairn::gemm

// 32 columns and four waves a workgroup: n / 32 workgroups, each wave a quarter of k.
hipError_t cairn_skinny(const cairn::gemm::Params& p, hipStream_t s, int) {
  constexpr int GROUPS = 2, SPLIT = 4, UNROLL = 4;
  const dim3 grid(unsigned((p.n + 16 * GROUPS - 1) / (16 * GROUPS)));
  hipLaunchKernelGGL((cairn::gemm::skinny_gemm<GROUPS, SPLIT, UNROLL>), grid, dim3(64 * SPLIT), 0, s, p);
  return hipGetLastError();
}
