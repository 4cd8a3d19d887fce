// Device helpers of the LDS-ring GEMMs (wave.hpp) and the skinny ring (gemm_skinny.hip): the buffer resource and the 16-byte
// global-to-LDS load that fills the ring, the waits and barrier that order it, and the MFMA operand reads.
#pragma once
#include <hip/hip_runtime.h>
#include "pipe.hpp"
#include "tile.hpp"

namespace cairn::gemm {
using namespace cairn::pipe;
typedef unsigned su32x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef int i32x2 __attribute__((ext_vector_type(2)));

// The LDS address of a pointer into the workgroup's LDS.
__device__ inline unsigned lds_address(const char* p) {
  return unsigned(reinterpret_cast<std::uintptr_t>((const __attribute__((address_space(3))) char*)p));
}
#define LDS_PTR(p) ((__attribute__((address_space(3))) void*)(p))

__device__ inline __amdgpu_buffer_rsrc_t span_of(const char* base, std::int64_t bytes) {
  const std::int64_t capped = bytes < 0 ? 0 : (bytes > 0x7fffffffLL ? 0x7fffffffLL : bytes);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(base), (short)0, (int)capped, 0x00020000);
}

// The device's policy for Loader: a buffer resource (four SGPRs), and one 16-byte load per lane into LDS at the
// wave's base + 16 lane (the lane's own offset chooses what it fetches). The load is written out here, M0 set from a
// scalar, so that the compiler does not see LDS written behind its back and wait on every prefetch in flight before
// the LDS reads of a stage that has long landed; the kernel orders the prefetches itself (vmcnt waits and barriers).
struct Dma {
  using Rsrc = su32x4;
  __device__ static Rsrc resource(const char* base, std::int64_t bytes) {
    const std::int64_t capped = bytes < 0 ? 0 : (bytes > 0x7fffffffLL ? 0x7fffffffLL : bytes);
    const std::uint64_t addr = reinterpret_cast<std::uintptr_t>(base);
    return Rsrc{unsigned(addr), unsigned(addr >> 32) & 0xffffu, unsigned(capped), 0x00020000u};
  }
  __device__ static Rsrc resource(const char* at, unsigned records) {
    const std::uint64_t addr = reinterpret_cast<std::uintptr_t>(at);
    return Rsrc{unsigned(addr), unsigned(addr >> 32) & 0xffffu, records, 0x00020000u};
  }
  __device__ static Rsrc resource(const Walk& w) { return resource(w.at, w.records()); }
  __device__ static void load_lds(Rsrc r, unsigned lds_at, int offset) {
    const unsigned m0 = __builtin_amdgcn_readfirstlane(lds_at);
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds" ::"s"(m0), "v"(offset), "s"(r)
                 : "memory", "m0");
  }
  __device__ static void load_lds(Rsrc r, char* wave_base, int offset) { load_lds(r, lds_address(wave_base), offset); }
  // M0 once for several loads: the LDS base they share (each adds its immediate offset). Nothing else of the kernel
  // writes M0 (the LDS instructions of gfx950 do not use it), which a test of the compiled loop checks.
  __device__ static void set_base(unsigned lds_at) {
    const unsigned m0 = __builtin_amdgcn_readfirstlane(lds_at);
    asm volatile("s_mov_b32 m0, %0" ::"s"(m0) : "memory", "m0");
  }
  template<int U> __device__ static void load_lds_imm(Rsrc r, int offset) {
    asm volatile("buffer_load_dwordx4 %0, %1, 0 offen offset:%2 lds" ::"v"(offset - 1024 * U), "s"(r), "n"(1024 * U)
                 : "memory");
  }
};

// Wait until at most N of this wave's vector-memory operations are outstanding, then (barrier) until every wave
// of the workgroup has reached the same point with its LDS reads complete.
template<int N> __device__ inline void wait_loads() { asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory"); }
__device__ inline void barrier() { asm volatile("s_barrier" ::: "memory"); }

// One LDS transpose read: 8 bytes a lane, each lane one column of a 4 x 16 (16-bit) or 8 x 16 (byte) block that
// 16 lanes supply row-wise.
template<int ES> __device__ __forceinline__ u32x2 transpose_half(const char* at) {
  if constexpr(ES == 2)
    return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(at)));
  else
    return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr8_b64_v2i32((__attribute__((address_space(3))) i32x2*)(at)));
}

// The MFMA operands of one k-step s for COUNT 32-row blocks at row0 + 32 i of an operand held R rows wide: K-major,
// one ds_read_b128 each; M/N-major, two transpose reads each (k bytes 0-7, then 8-15 of the lane's 16).
template<class Sh, int R, bool KMAJOR, int COUNT>
__device__ inline void fragments(u32x4 (&out)[COUNT], const char* stage, int row0, int s, int l) {
  if constexpr(KMAJOR) {
#pragma unroll
    for(int i = 0; i < COUNT; ++i) out[i] = *reinterpret_cast<const u32x4*>(stage + kmajor_fragment(row0 + 32 * i, s, l));
  } else {
#pragma unroll
    for(int i = 0; i < COUNT; ++i) {
      u32x2 half[2];
#pragma unroll
      for(int h = 0; h < 2; ++h) {
        const char* at = stage + mnmajor_fragment<Sh::ES, R>(row0 + 32 * i, s, h, l);
        if constexpr(Sh::ES == 2)
          half[h] = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                                                  (__attribute__((address_space(3))) s16x4*)(at)));
        else
          half[h] = __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr8_b64_v2i32(
                                                  (__attribute__((address_space(3))) i32x2*)(at)));
      }
      out[i] = u32x4{half[0][0], half[0][1], half[1][0], half[1][1]};
    }
  }
}

}  // namespace cairn::gemm
