// The HIP machine's device code for gfx950 (the members cairn_hip.hpp declares): the lane kernels a generated
// program's regions run as, the fill that writes zeros, and the fold and inclusive scan the context's reductions,
// scans and compactions queue.
//
// Regions. A region's indices are dealt out grid-stride, so every index below n runs exactly once whatever block and
// indices a lane a plan chose. A block is 256 threads (four 64-wide waves) unless the plan asks otherwise, clipped to
// what the kernel's registers allow in whole waves. A staged plan's tile lives in LDS, up to the CU's 160 KiB (past
// 64 KiB the kernel is told first).
//
// Folds and scans are deterministic: for a given n the association is fixed, so two runs give the same bits, and no
// atomics are used. The first pass deals [0, n) out in equal runs, one a block (fold_blocks(n) blocks, at most 1024,
// each run at least 8192 indices); a block's 256 lanes fold their run's indices strided by 256, then a tree in LDS
// folds the 256 partials. A fold then folds the blocks' partials the same way in one block. A scan also scans the
// partials (one block), then scans each run again tile by tile (256 indices, a tree scan in LDS), starting from the
// total of the runs before it, into `out`. value(i) must not depend on the order it is evaluated in; a scan
// evaluates it twice.
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>
#include <type_traits>
#include "cairn_hip.hpp"

namespace cr::gpu {

constexpr unsigned WAVE = 64;
constexpr unsigned MAX_GRID = 65535;  // blocks a region asks for at most; the grid-stride loop covers the rest

namespace kernels {

template<unsigned U, class F> __global__ void lanes(std::size_t n, F body) {
  const std::size_t stride = std::size_t(gridDim.x) * blockDim.x;
  std::size_t i = std::size_t(blockIdx.x) * blockDim.x + threadIdx.x;
#pragma unroll U
  for(; i < n; i += stride) body(i);
}

// W adjacent indices a lane over whole W-wide chunks; indices past the last whole chunk one at a time.
template<unsigned W, unsigned U, class F, class G> __global__ void chunks(std::size_t n, F scalar, G chunk) {
  const std::size_t stride = std::size_t(gridDim.x) * blockDim.x * W;
  std::size_t i = (std::size_t(blockIdx.x) * blockDim.x + threadIdx.x) * W;
#pragma unroll U
  for(; i < n; i += stride) {
    if(i + W <= n) chunk(i);
    else
      for(std::size_t j = i; j < n; ++j) scalar(j);
  }
}

// A block's tiles of blockDim.x indices from `base`: each loaded into LDS with R halo elements a side, between two
// barriers every thread of the block reaches, then run.
template<std::size_t R, unsigned U, class L, class F> __global__ void staged(std::size_t n, L load, F body) {
  extern __shared__ __attribute__((aligned(16))) unsigned char tile[];
  const std::size_t width = blockDim.x, halo = width + 2 * R, t = threadIdx.x;
  const std::size_t stride = std::size_t(gridDim.x) * width;
  std::size_t base = std::size_t(blockIdx.x) * width;
#pragma unroll U
  for(; base < n; base += stride) {
    __syncthreads();  // every thread is done with the previous tile
    load(base, halo, t, width, tile);
    __syncthreads();
    if(base + t < n) body(base + t, base, halo, tile);
  }
}

// Zeros: 16 bytes a lane over the aligned words, then the bytes past them.
__global__ void zero_words(uint4* p, std::size_t words) {
  const std::size_t stride = std::size_t(gridDim.x) * blockDim.x;
  for(std::size_t i = std::size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < words; i += stride)
    p[i] = uint4{0u, 0u, 0u, 0u};
}
__global__ void zero_bytes(unsigned char* p, std::size_t bytes) {
  const std::size_t stride = std::size_t(gridDim.x) * blockDim.x;
  for(std::size_t i = std::size_t(blockIdx.x) * blockDim.x + threadIdx.x; i < bytes; i += stride) p[i] = 0;
}

constexpr unsigned FOLD_THREADS = 256;

// LDS for 256 (or 2 x 256) values of a trivially copyable T that need not be default-constructible.
template<class T, unsigned COUNT> struct Slots {
  alignas(T) unsigned char raw[COUNT * sizeof(T)];
  __device__ T& operator[](unsigned i) { return reinterpret_cast<T*>(raw)[i]; }
};

// The block's 256 values folded by a tree: lane t and t + s, s = 128, 64, .., 1. Every thread gets the result.
template<class T, class Op> __device__ T block_fold(T v, Op op, Slots<T, FOLD_THREADS>& s) {
  const unsigned t = threadIdx.x;
  s[t] = v;
  __syncthreads();
#pragma unroll
  for(unsigned half = FOLD_THREADS / 2; half > 0; half >>= 1) {
    if(t < half) s[t] = op(s[t], s[t + half]);
    __syncthreads();
  }
  const T r = s[0];
  __syncthreads();  // the slots may be reused
  return r;
}

// The block's 256 values scanned (inclusive) by doubling: after the step of distance d, slot t holds the fold of
// t - 2d + 1 .. t. Two buffers, one read and one written each step. Every thread gets its prefix; *total the last.
template<class T, class Op> __device__ T block_scan(T v, Op op, Slots<T, 2 * FOLD_THREADS>& s, T* total) {
  const unsigned t = threadIdx.x;
  unsigned from = 0;
  s[t] = v;
  __syncthreads();
#pragma unroll
  for(unsigned d = 1; d < FOLD_THREADS; d <<= 1) {
    const unsigned to = FOLD_THREADS - from;
    T x = s[from + t];
    if(t >= d) x = op(s[from + t - d], x);
    s[to + t] = x;
    from = to;
    __syncthreads();
  }
  const T r = s[from + t];
  *total = s[from + FOLD_THREADS - 1];
  __syncthreads();
  return r;
}

// One fold pass: block b folds value(i) for i in [b run, min(n, (b + 1) run)) into out[b].
template<class T, class F, class Op>
__global__ void __launch_bounds__(FOLD_THREADS) fold_runs(std::size_t n, std::size_t run, F value, Op op, T identity,
                                                          T* out) {
  __shared__ Slots<T, FOLD_THREADS> s;
  const std::size_t first = std::size_t(blockIdx.x) * run;
  const std::size_t last = first + run < n ? first + run : n;
  T acc = identity;
  for(std::size_t i = first + threadIdx.x; i < last; i += FOLD_THREADS) acc = op(acc, value(i));
  acc = block_fold(acc, op, s);
  if(threadIdx.x == 0) out[blockIdx.x] = acc;
}

// One scan pass: block b scans value(i) over its run, tile by tile, starting from carries[b - 1] (the fold of the
// runs before it; the identity for the first block or without carries), into out.
template<class T, class F, class Op>
__global__ void __launch_bounds__(FOLD_THREADS) scan_runs(std::size_t n, std::size_t run, F value, Op op, T identity,
                                                          const T* carries, T* out) {
  __shared__ Slots<T, 2 * FOLD_THREADS> s;
  const std::size_t first = std::size_t(blockIdx.x) * run;
  const std::size_t last = first + run < n ? first + run : n;
  T carry = carries && blockIdx.x ? carries[blockIdx.x - 1] : identity;
  for(std::size_t base = first; base < last; base += FOLD_THREADS) {
    const std::size_t i = base + threadIdx.x;
    T total;
    const T x = block_scan(i < last ? value(i) : identity, op, s, &total);
    if(i < last) out[i] = op(carry, x);
    carry = op(carry, total);
  }
}

// Element i of an array, as a value function.
template<class T> struct Element {
  const T* p;
  __device__ T operator()(std::size_t i) const { return p[i]; }
};

}  // namespace kernels

// The most threads a block of `kernel` holds, in whole waves (a planned block its registers cannot fill runs as wide
// as fits, and computes the same).
template<class K> inline unsigned widest(K kernel) noexcept {
  hipFuncAttributes held{};
  check(hipFuncGetAttributes(&held, reinterpret_cast<const void*>(kernel)));
  const unsigned most = unsigned(held.maxThreadsPerBlock) / WAVE * WAVE;
  return most ? most : WAVE;
}
inline unsigned blocks_for(std::size_t n, std::size_t each) noexcept {
  const std::size_t g = (n + each - 1) / each;
  return g < 1 ? 1u : (g < MAX_GRID ? unsigned(g) : MAX_GRID);
}
inline unsigned clipped(unsigned block, unsigned most) noexcept {
  if(!block) block = reuse::BLOCK;
  return block < most ? block : most;
}

template<unsigned U, class F>
inline void Hip::lanes(std::size_t n, const F& body, Stream s, unsigned block, std::size_t per_lane) noexcept {
  static_assert(std::is_trivially_copyable_v<F>, "a lane body crosses over as kernel arguments");
  if(!n) return;
  static const unsigned most = widest(kernels::lanes<U, F>);
  block = clipped(block, most);
  const std::size_t each = std::size_t(block) * (per_lane ? per_lane : 1);
  hipLaunchKernelGGL((kernels::lanes<U, F>), dim3(blocks_for(n, each)), dim3(block), 0, s, n, body);
  check(hipGetLastError());
}

template<unsigned W, unsigned U, class F, class G>
inline void Hip::vector_lanes(std::size_t n, F scalar, G chunk, Stream s, unsigned block,
                              std::size_t per_lane) noexcept {
  if(!n) return;
  static const unsigned most = widest(kernels::chunks<W, U, F, G>);
  block = clipped(block, most);
  const std::size_t each = std::size_t(block) * (per_lane ? per_lane : 1) * W;
  hipLaunchKernelGGL((kernels::chunks<W, U, F, G>), dim3(blocks_for(n, each)), dim3(block), 0, s, n, scalar, chunk);
  check(hipGetLastError());
}

template<std::size_t R, unsigned U, class L, class F, class S>
inline void Hip::staged_lanes(std::size_t n, L load, F body, S bytes, Stream s, unsigned block,
                              std::size_t per_lane) noexcept {
  if(!n) return;
  static const unsigned most = widest(kernels::staged<R, U, L, F>);
  block = clipped(block, most);
  const std::size_t lds = bytes(std::size_t(block) + 2 * R);
  if(lds > 160 * 1024) trap();  // more than a CU holds
  if(lds > 64 * 1024)
    check(hipFuncSetAttribute(reinterpret_cast<const void*>(kernels::staged<R, U, L, F>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, int(lds)));
  const std::size_t each = std::size_t(block) * (per_lane ? per_lane : 1);
  hipLaunchKernelGGL((kernels::staged<R, U, L, F>), dim3(blocks_for(n, each)), dim3(block), unsigned(lds), s, n, load,
                     body);
  check(hipGetLastError());
}

inline void Hip::zero(void* p, std::size_t bytes, Stream s) noexcept {
  if(!bytes) return;
  unsigned char* c = static_cast<unsigned char*>(p);
  std::size_t words = 0;
  if(reinterpret_cast<std::uintptr_t>(c) % 16 == 0) {
    words = bytes / 16;
    if(words) {
      hipLaunchKernelGGL(kernels::zero_words, dim3(blocks_for(words, 1024)), dim3(256), 0, s,
                         reinterpret_cast<uint4*>(c), words);
      check(hipGetLastError());
    }
  }
  if(bytes > 16 * words) {
    hipLaunchKernelGGL(kernels::zero_bytes, dim3(blocks_for(bytes - 16 * words, 1024)), dim3(256), 0, s,
                       c + 16 * words, bytes - 16 * words);
    check(hipGetLastError());
  }
}

template<class T, class F, class Op>
inline void Hip::fold(std::size_t n, F value, Op op, T identity, T* out, void* work, Stream s) noexcept {
  static_assert(std::is_trivially_copyable_v<T> && std::is_trivially_copyable_v<F>, "crosses as kernel arguments");
  const unsigned g = fold_blocks(n);
  const std::size_t run = (n + g - 1) / g;
  T* partial = static_cast<T*>(work);
  hipLaunchKernelGGL((kernels::fold_runs<T, F, Op>), dim3(g), dim3(kernels::FOLD_THREADS), 0, s, n, run, value, op,
                     identity, partial);
  check(hipGetLastError());
  hipLaunchKernelGGL((kernels::fold_runs<T, kernels::Element<T>, Op>), dim3(1), dim3(kernels::FOLD_THREADS), 0, s,
                     std::size_t(g), std::size_t(g), kernels::Element<T>{partial}, op, identity, out);
  check(hipGetLastError());
}

template<class T, class F, class Op>
inline void Hip::scan(std::size_t n, F value, Op op, T identity, T* out, void* work, Stream s) noexcept {
  static_assert(std::is_trivially_copyable_v<T> && std::is_trivially_copyable_v<F>, "crosses as kernel arguments");
  if(!n) return;
  const unsigned g = fold_blocks(n);
  const std::size_t run = (n + g - 1) / g;
  T* partial = static_cast<T*>(work);
  T* carries = partial + g;
  hipLaunchKernelGGL((kernels::fold_runs<T, F, Op>), dim3(g), dim3(kernels::FOLD_THREADS), 0, s, n, run, value, op,
                     identity, partial);
  check(hipGetLastError());
  hipLaunchKernelGGL((kernels::scan_runs<T, kernels::Element<T>, Op>), dim3(1), dim3(kernels::FOLD_THREADS), 0, s,
                     std::size_t(g), std::size_t(g), kernels::Element<T>{partial}, op, identity,
                     static_cast<const T*>(nullptr), carries);
  check(hipGetLastError());
  hipLaunchKernelGGL((kernels::scan_runs<T, F, Op>), dim3(g), dim3(kernels::FOLD_THREADS), 0, s, n, run, value, op,
                     identity, static_cast<const T*>(carries), out);
  check(hipGetLastError());
}

}  // namespace cr::gpu
