// The tiled MFMA GEMM for gfx950: bf16/f16 on v_mfma_f32_32x32x16_{bf16,f16}, int8 on v_mfma_i32_32x32x32_i8, and
// the 8-bit floats widened to f16 on their way into LDS (tile.hpp, widened) and multiplied as f16. The f16 matrix
// core's products of widened 8-bit floats are exact and their sums f32-rounded, which keeps the multiply's contract;
// the 8-bit float matrix core (the ring kernels' wave8 form) does not at short k: it adds its products in groups
// with a narrower alignment.
//
// One workgroup of four waves computes one BM x BN output tile (up to 256 x 256), walking k in steps of 128 bytes
// of every operand row. Both operands sit K-major in LDS, two stages deep (up to 128 KiB of the CU's 160 KiB), each
// 128-byte row XOR-swizzled in 16-byte chunks (tile.hpp). A K-contiguous operand (A of NN/NT, B of NT/TT) crosses
// in 16-byte buffer loads, 8 threads to a row; an M- or N-contiguous one (B of NN, A of TN) crosses as blocks of
// 8 columns x 8 (bf16) or 16 (int8) k rows that each thread transposes in registers before writing K-major chunks.
// While the waves multiply stage s the next stage's loads are in flight; one barrier per k-step.
//
// Buffer loads return zero past the matrix (rows past m or n, k past k), so edge tiles need no branch and the zero
// rows add 0 * 0 to outputs that are never written. The output crosses straight from the accumulators: each lane
// holds four consecutive columns of a row per register quad, stored as 16 (f32, int32) or 8 (bf16/f16) bytes.
//
// The reference runs a fixed 64 x 64 WMMA tiling in two stages (src/cairn/runtime/cairn_tensor.hpp:145-196); this is
// its gfx950 replacement, sized for 256 CUs of 160 KiB LDS and a 64-wide wave.
#include <hip/hip_runtime.h>
#include "kernels.hpp"
#include "mfma.hpp"
#include "tile.hpp"

namespace cairn::gemm {
using namespace cairn::tile;

// The device's memory policy for Operand: buffer loads, which return zero past the resource.
struct Buffer {
  using Rsrc = __amdgpu_buffer_rsrc_t;
  __device__ static Rsrc resource(const char* base, std::int64_t bytes) {
    const std::int64_t capped = bytes < 0 ? 0 : (bytes > 0x7fffffffLL ? 0x7fffffffLL : bytes);
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(base), (short)0, (int)capped, 0x00020000);
  }
  __device__ static u32x4 load16(Rsrc r, int offset) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(r, offset, 0, 0));
  }
  __device__ static u32x2 load8(Rsrc r, int offset) {
    return __builtin_bit_cast(u32x2, __builtin_amdgcn_raw_buffer_load_b64(r, offset, 0, 0));
  }
};
// LDS for Operand::store.
struct Shared {
  char* base;
  __device__ void write16(int offset, u32x4 v) { *reinterpret_cast<u32x4*>(base + offset) = v; }
};

template<class Sh, int OP, bool TA, bool TB>
__global__ void __launch_bounds__(256) mfma_gemm(Params p) {
  using M = Mfma<Sh::W == WIDEN_NONE ? OP : int(OP_F16)>;
  using Acc = typename M::Acc;
  constexpr bool A_KMAJOR = !TA, B_KMAJOR = TB;
  __shared__ __attribute__((aligned(16))) char lds[2 * Sh::STAGE];

  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const int wm = wave / Sh::WAVES_N, wn = wave % Sh::WAVES_N;
  int tm, tn;
  tile_of(int(blockIdx.x), p.tiles_m, p.tiles_n, p.group, tm, tn);
  const int row0 = tm * Sh::BM, col0 = tn * Sh::BN;

  const char* a = static_cast<const char*>(p.a);
  const char* b = static_cast<const char*>(p.b);
  const Panel pa = panel(A_KMAJOR, row0, p.m, p.k, p.lda, Sh::GS);
  const Panel pb = panel(B_KMAJOR, col0, p.n, p.k, p.ldb, Sh::GS);
  Buffer mem;
  Shared shared{lds};
  Operand<Sh, Sh::BM, A_KMAJOR, Buffer> fa;
  Operand<Sh, Sh::BN, B_KMAJOR, Buffer> fb;
  fa.setup(t, row0, p.m, p.lda);
  fb.setup(t, col0, p.n, p.ldb);
  auto fetch = [&](int kt) {
    fa.fetch(mem, a, pa, p.lda, kt, p.k, t);
    fb.fetch(mem, b, pb, p.ldb, kt, p.k, t);
  };
  auto store = [&](int s) {
    fa.store(shared, s * Sh::STAGE, t);
    fb.store(shared, s * Sh::STAGE + Sh::A_BYTES, t);
  };

  Acc acc[Sh::FM][Sh::FN];
#pragma unroll
  for(int i = 0; i < Sh::FM; ++i)
#pragma unroll
    for(int j = 0; j < Sh::FN; ++j) acc[i][j] = Acc{};

  const int steps = (p.k + Sh::BK - 1) / Sh::BK;
  if(steps > 0) {
    fetch(0);
    store(0);
  }
  __syncthreads();
  for(int kt = 0; kt < steps; ++kt) {
    const bool more = kt + 1 < steps;
    if(more) fetch(kt + 1);
    const char* sa = lds + (kt & 1) * Sh::STAGE;
    const char* sb = sa + Sh::A_BYTES;
#pragma unroll
    for(int s = 0; s < Sh::STEPS; ++s) {
      u32x4 xa[Sh::FM], xb[Sh::FN];
#pragma unroll
      for(int i = 0; i < Sh::FM; ++i)
        xa[i] = *reinterpret_cast<const u32x4*>(sa + fragment_offset(wm * Sh::WTM + 32 * i, s, lane));
#pragma unroll
      for(int j = 0; j < Sh::FN; ++j)
        xb[j] = *reinterpret_cast<const u32x4*>(sb + fragment_offset(wn * Sh::WTN + 32 * j, s, lane));
#pragma unroll
      for(int i = 0; i < Sh::FM; ++i)
#pragma unroll
        for(int j = 0; j < Sh::FN; ++j) acc[i][j] = M::step(xb[j], xa[i], acc[i][j]);
    }
    if(more) store((kt + 1) & 1);
    __syncthreads();
  }

  // Epilogue: register quad q of block (i, j) is row m, columns n .. n+3.
  char* c = static_cast<char*>(p.c);
#pragma unroll
  for(int i = 0; i < Sh::FM; ++i) {
    const int m = row0 + wm * Sh::WTM + 32 * i + acc_m(lane);
#pragma unroll
    for(int j = 0; j < Sh::FN; ++j)
#pragma unroll
      for(int q = 0; q < 4; ++q) {
        const int n = col0 + wn * Sh::WTN + 32 * j + acc_n(lane, q);
        if(m >= p.m || n >= p.n) continue;
        const std::int64_t at = std::int64_t(m) * p.ldc + n;
        if(OP == OP_I8 && p.c_type == CAIRN_TYPE_I32) {
          i32x4 w;
#pragma unroll
          for(int e = 0; e < 4; ++e) w[e] = int(acc[i][j][4 * q + e]);
          *reinterpret_cast<i32x4*>(c + at * 4) = w;
          continue;
        }
        float v[4];
#pragma unroll
        for(int e = 0; e < 4; ++e) v[e] = float(acc[i][j][4 * q + e]);
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
  }
}

// The launcher for one instance: a tile per workgroup.
template<class Sh, int OP, bool TA, bool TB> hipError_t launch(const Params& p, hipStream_t s) {
  const unsigned grid = unsigned(p.tiles_m) * unsigned(p.tiles_n);
  hipLaunchKernelGGL((mfma_gemm<Sh, OP, TA, TB>), dim3(grid), dim3(256), 0, s, p);
  return hipGetLastError();
}

}  // namespace cairn::gemm

// The instances the kernel table (capi.cpp) names: int8 one byte to an element in LDS, the 8-bit floats widened.
namespace cairn::gemm {
constexpr int widen_of(int op) {
  return op == OP_F8E4M3 ? tile::WIDEN_E4M3 : (op == OP_F8E5M2 ? tile::WIDEN_E5M2 : tile::WIDEN_NONE);
}
}  // namespace cairn::gemm
#define CAIRN_MFMA_INSTANCE(NAME, BM, BN, OP, TA, TB)                                                             \
  hipError_t NAME(const cairn::gemm::Params& p, hipStream_t s) {                                                 \
    using Sh = cairn::tile::Shape<BM, BN, (OP == cairn::gemm::OP_I8 ? 1 : 2), cairn::gemm::widen_of(OP)>;        \
    return cairn::gemm::launch<Sh, OP, TA, TB>(p, s);                                                            \
  }
#include "instances.inc"
