// A clock-stamp build of the ring GEMM (cairn_amd/csrc/wave.hpp) for `bench.py --only stamps`: the library's whole-
// tile kernel with a Clock that reads the reference clock (s_memrealtime, 100 MHz, one count across the chip) and the
// shader clock (s_memtime, the XCD's own) at five points of each wave's tile, and writes them with the wave's XCD and
// tile after its last store has completed. Square NN problems of one round (n a multiple of 256, the tile count a
// multiple of the 8 XCDs), bf16 out: the bf16 GEMM of C2 and the int8 W8A8 GEMM of C4 with its dequant.
//
// Record of wave w of workgroup b: 16 values at stamps + 16 (4 b + w): [0, 5) reference clock at points 0 .. 4 (start,
// first MFMA, main loop done, stores issued, stores done), [5, 10) shader clock at the same points, 10 the XCD, 11 the
// hardware id register, 12 and 13 the tile.
#include "../../cairn_amd/csrc/wave.hpp"

namespace {
using cairn::gemm::Params;

struct Stamps {
  static constexpr bool on = true;
  unsigned long long real[5], shader[5];
  template<int POINT> __device__ __forceinline__ void mark() {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // the clock reads below are the only scalar reads in flight
    real[POINT] = __builtin_amdgcn_s_memrealtime();
    shader[POINT] = __builtin_amdgcn_s_memtime();
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  }
  __device__ __forceinline__ void record(const Params& p, int tm, int tn, int wave, int lane) {
    if(lane != 0) return;
    unsigned long long* o = static_cast<unsigned long long*>(p.work) + (std::size_t(blockIdx.x) * 4 + wave) * 16;
#pragma unroll
    for(int i = 0; i < 5; ++i) {
      o[i] = real[i];
      o[5 + i] = shader[i];
    }
    o[10] = __builtin_amdgcn_s_getreg(20 | (15 << 11));  // HW_REG_XCC_ID, bits 0 .. 15
    o[11] = __builtin_amdgcn_s_getreg(4 | (31 << 11));   // HW_REG_HW_ID, all 32 bits
    o[12] = unsigned(tm);
    o[13] = unsigned(tn);
  }
};

template<class Sh, int OP, bool RAW> __global__ void __launch_bounds__(256) clocked(Params p) {
  CAIRN_WAVE_LDS(Sh)
  int tm, tn;
  cairn::tile::tile_at(cairn::tile::whole_id(p.split, int(blockIdx.x)), p.tiles_m, p.tiles_n, p.group, tm, tn);
  cairn::gemm::wave_tile<Sh, OP, false, false, RAW, false, Stamps>(p, lds, terms, tm, tn, 0, p.k, nullptr);
}

// The parameters capi.cpp gives a square NN problem of one round of whole tiles: tile ids dealt to the 8 XCDs in
// blocks, no split.
bool square(Params& p, const void* a, const void* b, void* c, void* stamps, int n, int type, const float* rs,
            const float* cs) {
  if(n <= 0 || n % 256 || (n / 256) * (n / 256) % 8) return false;
  p = Params{};
  p.a = a;
  p.b = b;
  p.c = c;
  p.lda = p.ldb = p.ldc = n;
  p.m = p.n = p.k = n;
  p.tiles_m = p.tiles_n = n / 256;
  p.group = 4;
  p.a_type = type;
  p.c_type = CAIRN_TYPE_BF16;
  p.act = CAIRN_ACT_NONE;
  p.bias_type = CAIRN_TYPE_F32;
  p.row_scale = rs;
  p.col_scale = cs;
  p.rows16 = (reinterpret_cast<std::uintptr_t>(c) % 16) == 0;
  p.whole_tiles = p.tiles_m * p.tiles_n;
  p.split.xcds = 8;
  p.split.block = p.whole_tiles / 8;
  p.split.first = p.split.block;
  p.work = stamps;
  return true;
}
}  // namespace

// bf16 a, b (n x n), bf16 c; stamps: 4 * 16 * (n / 256)^2 values of 8 bytes.
extern "C" int wave_stamps_bf16(const void* a, const void* b, void* c, void* stamps, int n, hipStream_t s) {
  Params p;
  if(!square(p, a, b, c, stamps, n, CAIRN_TYPE_BF16, nullptr, nullptr)) return int(hipErrorInvalidValue);
  hipLaunchKernelGGL((clocked<cairn::pipe::Shape<256, 256, 2, 4, 4>, cairn::gemm::OP_BF16, false>),
                     dim3(unsigned(p.whole_tiles)), dim3(256), 0, s, p);
  return int(hipGetLastError());
}

// int8 a, b with f32 row and column scales (the W8A8 dequant), bf16 c.
extern "C" int wave_stamps_i8(const void* a, const void* b, void* c, const float* rs, const float* cs, void* stamps,
                              int n, hipStream_t s) {
  Params p;
  if(!square(p, a, b, c, stamps, n, CAIRN_TYPE_I8, rs, cs)) return int(hipErrorInvalidValue);
  hipLaunchKernelGGL((clocked<cairn::pipe::Shape<256, 256, 1, 4, 4>, cairn::gemm::OP_I8, false>),
                     dim3(unsigned(p.whole_tiles)), dim3(256), 0, s, p);
  return int(hipGetLastError());
}
