// Device regions on the HIP machine: the lane kernels a generated program's `parallel`, `plan vector` and `plan stage`
// regions run as (the role of src/cairn/runtime/cairn_kernels.hpp:60-140), the device library's reduce and scans on
// hipCUB (cairn_cub.hpp's), and the operations generated code calls on the thread's context (cairn_exec.hpp:25-230):
// scoped owners of device, pinned and unified storage, `run` and its vector and staged plans, `transfer`, reductions,
// scans, compaction and queued work on lent lanes. Built by hipcc for gfx950; a lane body is a __device__ lambda or
// any trivially copyable functor.
//
// On gfx950 a launch's block is 256 threads (four 64-wide waves) unless a plan asks otherwise, clipped to what the
// kernel's registers allow in whole waves; a region's indices are spread grid-stride, so every index below n runs
// exactly once whatever the block and the indices per thread chosen. A staged plan's tile lives in LDS (up to the
// CU's 160 KiB; past 64 KiB the kernel is told so first).
#pragma once
#include <hip/hip_runtime.h>
#include <hipcub/hipcub.hpp>
#include <cstring>
#include <iterator>
#include <type_traits>
#include "cairn_hip.hpp"

namespace cr::gpu {

constexpr unsigned WAVE = 64;
constexpr unsigned MAX_GRID = 65535;  // blocks a lane launch asks for at most; the grid-stride loop covers the rest

namespace lane_kernels {

template<unsigned U, class F> __global__ void lanes(std::size_t n, F body) {
  const std::size_t step = std::size_t(gridDim.x) * blockDim.x;
#pragma unroll U
  for(std::size_t i = blockIdx.x * std::size_t(blockDim.x) + threadIdx.x; i < n; i += step) body(i);
}

// W adjacent indices a thread over whole chunks; the last indices past a whole chunk one at a time.
template<unsigned W, unsigned U, class F, class G> __global__ void chunks(std::size_t n, F scalar, G chunk) {
  const std::size_t step = std::size_t(gridDim.x) * blockDim.x * W;
#pragma unroll U
  for(std::size_t i = (blockIdx.x * std::size_t(blockDim.x) + threadIdx.x) * W; i < n; i += step) {
    if(n - i >= W) chunk(i);
    else
      for(std::size_t k = i; k < n; ++k) scalar(k);
  }
}

// A block's tiles of blockDim.x indices from `base`, each loaded into LDS (with R halo elements either side) between
// two barriers every thread of the block reaches, then run.
template<std::size_t R, unsigned U, class L, class F> __global__ void staged(std::size_t n, L load, F body) {
  extern __shared__ __attribute__((aligned(16))) unsigned char tile[];
  const std::size_t b = blockDim.x, w = b + 2 * R, t = threadIdx.x, step = std::size_t(gridDim.x) * b;
#pragma unroll U
  for(std::size_t base = blockIdx.x * b; base < n; base += step) {
    __syncthreads();  // the block is done with the last tile before this one overwrites it
    load(base, w, t, b, tile);
    __syncthreads();
    if(base + t < n) body(base + t, base, w, tile);
  }
}

}  // namespace lane_kernels

// The most threads a block of `kernel` can hold, in whole waves (a planned block its registers cannot fill runs as
// wide as fits and computes the same).
template<class K> inline unsigned widest(K kernel) noexcept {
  hipFuncAttributes held{};
  check(hipFuncGetAttributes(&held, reinterpret_cast<const void*>(kernel)));
  const unsigned most = unsigned(held.maxThreadsPerBlock) / WAVE * WAVE;
  return most ? most : WAVE;
}
inline unsigned grid_for(std::size_t n, std::size_t each) noexcept {
  const std::size_t g = (n + each - 1) / each;
  return g < MAX_GRID ? unsigned(g ? g : 1) : MAX_GRID;
}
inline unsigned clip(unsigned block, unsigned most) noexcept {
  if(block > most) block = most;
  return block ? block : WAVE;
}

template<unsigned U, class F>
inline void Hip::lanes(std::size_t n, const F& body, Stream s, unsigned block, std::size_t per_lane) noexcept {
  static_assert(std::is_trivially_copyable_v<F>, "a lane body crosses over as kernel arguments");
  if(!n) return;
  static const unsigned most = widest(lane_kernels::lanes<U, F>);
  block = clip(block, most);
  hipLaunchKernelGGL((lane_kernels::lanes<U, F>), dim3(grid_for(n, std::size_t(block) * (per_lane ? per_lane : 1))),
                     dim3(block), 0, s, n, body);
  check(hipGetLastError());
}

template<unsigned W, unsigned U, class F, class G>
inline void Hip::vector_lanes(std::size_t n, F scalar, G chunk, Stream s, unsigned block,
                              std::size_t per_lane) noexcept {
  if(!n) return;
  static const unsigned most = widest(lane_kernels::chunks<W, U, F, G>);
  block = clip(block, most);
  hipLaunchKernelGGL((lane_kernels::chunks<W, U, F, G>),
                     dim3(grid_for(n, std::size_t(block) * (per_lane ? per_lane : 1) * W)), dim3(block), 0, s, n,
                     scalar, chunk);
  check(hipGetLastError());
}

template<std::size_t R, unsigned U, class L, class F, class S>
inline void Hip::staged_lanes(std::size_t n, L load, F body, S bytes, Stream s, unsigned block,
                              std::size_t per_lane) noexcept {
  if(!n) return;
  static const unsigned most = widest(lane_kernels::staged<R, U, L, F>);
  block = clip(block, most);
  const std::size_t shared = bytes(std::size_t(block) + 2 * R);
  if(shared > 160 * 1024) trap();  // more than a CU's LDS
  if(shared > 64 * 1024)           // past the default, the kernel must be told its dynamic LDS first
    check(hipFuncSetAttribute(reinterpret_cast<const void*>(lane_kernels::staged<R, U, L, F>),
                              hipFuncAttributeMaxDynamicSharedMemorySize, int(shared)));
  hipLaunchKernelGGL((lane_kernels::staged<R, U, L, F>), dim3(grid_for(n, std::size_t(block) * (per_lane ? per_lane : 1))),
                     dim3(block), unsigned(shared), s, n, load, body);
  check(hipGetLastError());
}

inline void Hip::zero(void* p, std::size_t b, Stream s) noexcept {
  if(!b) return;
  unsigned char* c = static_cast<unsigned char*>(p);
  std::size_t done = 0;
  if(reinterpret_cast<std::uintptr_t>(c) % 16 == 0) {  // 16 bytes a lane, then the tail's bytes
    uint4* w = reinterpret_cast<uint4*>(c);
    const std::size_t words = b / 16;
    if(words) lanes<1>(words, [=] __device__(std::size_t i) { w[i] = uint4{0u, 0u, 0u, 0u}; }, s, reuse::BLOCK, 4);
    done = words * 16;
  }
  if(done < b) lanes<1>(b - done, [=] __device__(std::size_t i) { c[done + i] = 0; }, s, reuse::BLOCK, 1);
}

template<class In, class Out, class Fold, class T>
inline void Hip::reduce(void* temp, std::size_t& bytes, In in, Out out, std::size_t n, Fold fold, T identity,
                        Stream s) noexcept {
  check(hipcub::DeviceReduce::Reduce(temp, bytes, in, out, n, fold, identity, s));
}
template<class In, class Out, class Fold>
inline void Hip::inclusive_scan(void* temp, std::size_t& bytes, In in, Out out, Fold fold, std::size_t n,
                                Stream s) noexcept {
  check(hipcub::DeviceScan::InclusiveScan(temp, bytes, in, out, fold, n, s));
}
// The library sums in its input's type; the input is read as the output's type, so byte flags summed into
// std::size_t offsets never wrap.
template<class In, class Out>
inline void Hip::exclusive_sum(void* temp, std::size_t& bytes, In in, Out out, std::size_t n, Stream s) noexcept {
  using V = typename std::iterator_traits<Out>::value_type;
  struct Widen {
    In in;
    __host__ __device__ V operator()(std::size_t i) const { return V(in[i]); }
  };
  const reuse::Indexed<V, Widen> wide{Widen{in}};
  check(hipcub::DeviceScan::ExclusiveSum(temp, bytes, wide, out, n, s));
}

// Scoped owners: zero-initialized storage of n elements, released at scope exit, never copied or moved. Device and
// unified storage is zeroed on the thread's synchronous lane, which is waited for; pinned storage on the host.
template<class T, Where W> class Owner final {
  T* p_ = nullptr;

public:
  explicit Owner(std::size_t n) noexcept {
    static_assert(std::is_trivially_copyable_v<T>, "zeroed bytes are a value");
    const std::size_t b = reuse::span<T>(n);
    if(!b) return;
    Context& ctx = here();
    ctx.observed();
    p_ = static_cast<T*>(ctx.api().allocate(W, b));
    if constexpr(W == Where::pinned) std::memset(p_, 0, b);
    else reuse::observed(ctx, [&](hipStream_t s) { ctx.api().zero(p_, b, s); });
  }
  ~Owner() noexcept {
    if(!p_) return;
    Context& ctx = here();
    ctx.observed();  // nothing still queued may reach the storage once it goes
    ctx.api().release(W, p_);
  }
  Owner(const Owner&) = delete;
  Owner& operator=(const Owner&) = delete;
  Owner(Owner&&) = delete;
  Owner& operator=(Owner&&) = delete;
  T* data() const noexcept { return p_; }
};
template<class T> using Buffer = Owner<T, Where::device>;
template<class T> using Pinned = Owner<T, Where::pinned>;
template<class T> using Unified = Owner<T, Where::unified>;

// `parallel i in n`: body(i) for every i below n, on the context's synchronous lane; returns once it has run.
template<unsigned U = 1, class F>
inline void run(Context& ctx, std::size_t n, F body, unsigned block = reuse::BLOCK, std::size_t per_lane = 1) noexcept {
  static_assert(std::is_trivially_copyable_v<F>, "a lane body crosses over as kernel arguments");
  if(!n) return;
  reuse::synchronous(ctx, [&](hipStream_t s) { ctx.api().template lanes<U>(n, body, s, block, per_lane); });
}

// `plan vector W`: a W-wide chunk of each array a lane touches only at [i], one aligned access each; `whole` (every
// chunked pointer on its chunk's width) decides for the whole region, else the scalar lanes run.
template<class T, unsigned W> struct alignas(sizeof(T) * W) Chunk final {
  static_assert((sizeof(T) * W & (sizeof(T) * W - 1)) == 0 && sizeof(T) * W <= 16, "one access of 16 bytes at most");
  T v[W];
  CR_HD static Chunk load(const T* p) noexcept { return *reinterpret_cast<const Chunk*>(p); }
  CR_HD void store(T* p) const noexcept { *reinterpret_cast<Chunk*>(p) = *this; }
  CR_HD T& operator[](unsigned k) noexcept { return v[k]; }
};
template<unsigned W, class... T> inline bool aligned(const T*... p) noexcept {
  return ((reinterpret_cast<std::uintptr_t>(p) % (sizeof(T) * W) == 0) && ...);
}
template<unsigned W, unsigned U = 1, class F, class G>
inline void run_vector(Context& ctx, std::size_t n, bool whole, F scalar, G chunk, unsigned block = reuse::BLOCK,
                       std::size_t per_lane = 1) noexcept {
  static_assert(std::is_trivially_copyable_v<F> && std::is_trivially_copyable_v<G>, "lanes cross as arguments");
  if(!whole) return run<U>(ctx, n, scalar, block, per_lane);
  if(!n) return;
  reuse::synchronous(ctx, [&](hipStream_t s) { ctx.api().template vector_lanes<W, U>(n, scalar, chunk, s, block, per_lane); });
}

// `plan stage R`: tiles of the block's width with R halo elements either side in LDS; `bytes(width)` is the LDS the
// staged arrays take for a tile of `width` elements.
template<class T> CR_HD constexpr std::size_t tile_bytes(std::size_t width) noexcept {
  return (width * sizeof(T) + 15) / 16 * 16;
}
template<std::size_t R, unsigned U = 1, class L, class F, class S>
inline void run_staged(Context& ctx, std::size_t n, L load, F body, S bytes, unsigned block = reuse::BLOCK,
                       std::size_t per_lane = 1) noexcept {
  static_assert(std::is_trivially_copyable_v<L> && std::is_trivially_copyable_v<F>, "lanes cross as arguments");
  if(!n) return;
  reuse::synchronous(ctx, [&](hipStream_t s) {
    ctx.api().template staged_lanes<R, U>(n, load, body, bytes, s, block, per_lane);
  });
}

// `transfer(dst, src)`: n elements on the context's stream. Between device views it is device work like a region;
// to or from host memory it is waited for, held or not.
template<class T> inline void copy_on(Context& ctx, T* dst, const T* src, std::size_t n, Dir d) noexcept {
  if(!n) return;
  auto queue = [&](hipStream_t s) { ctx.api().copy(dst, src, reuse::span<T>(n), d, s); };
  if(d == Dir::d2d) reuse::synchronous(ctx, queue);
  else reuse::observed(ctx, queue);
}

// Reductions and scans on the thread's context, whose budget has no limit: an over_budget answer would be a failed
// allocation, and traps.
template<class T, class Op, class F> inline T reduce_on(Context& ctx, std::size_t n, T identity, Op op, F value) noexcept {
  T result = identity;
  if(reuse::reduce(ctx, result, n, identity, op, value) != Scratch::ok) trap();
  return result;
}
template<bool Exclusive, class T, class R, class Op, class F>
inline T scan_on(Context& ctx, R* out, std::size_t n, T identity, Op op, F value) noexcept {
  T total = identity;
  if(reuse::scan<Exclusive>(ctx, total, out, n, identity, op, value) != Scratch::ok) trap();
  return total;
}
template<class T, class R, class Op, class F>
inline void reduce_into(Context& ctx, R* at, std::size_t n, T identity, Op op, F value) noexcept {
  if(reuse::reduce_into(ctx, at, n, identity, op, value) != Scratch::ok) trap();
}
template<bool Exclusive, class T, class R, class Op, class F>
inline void scan_into(Context& ctx, R* out, std::size_t n, T identity, Op op, F value) noexcept {
  if(reuse::scan_into<Exclusive>(ctx, out, n, identity, op, value) != Scratch::ok) trap();
}
template<class T, class P, class F>
inline std::size_t compact_on(Context& ctx, T* out, std::size_t n, P pred, F value) noexcept {
  std::size_t used = 0;
  if(reuse::compact(ctx, &used, out, n, pred, value) != Scratch::ok) trap();
  return used;
}

// Queued work (`spawn parallel ... after t`, `spawn transfer`): on a lent lane, after the tickets `after...`,
// returned at once; the lane comes back at the ticket's wait.
template<class F, class... After> inline Lent queue(Context& ctx, std::size_t n, F body, const After&... after) noexcept {
  static_assert(std::is_trivially_copyable_v<F>, "a lane body crosses over as kernel arguments");
  ctx.observed();
  Lent t(ctx);
  (t.follow(after.mark()), ...);
  if(n) ctx.api().template lanes<1>(n, body, t.stream(), reuse::BLOCK, 1);
  return t;
}
template<class T, class... After>
inline Lent queue_copy(Context& ctx, T* dst, const T* src, std::size_t n, Dir d, const After&... after) noexcept {
  ctx.observed();
  Lent t(ctx);
  (t.follow(after.mark()), ...);
  if(n) ctx.api().copy(dst, src, reuse::span<T>(n), d, t.stream());
  return t;
}
inline void wait(Lent&& t) noexcept { std::move(t).wait(); }

// The context API for a program or a test with a context of its own and a budget it declares.
template<class F, class... After> inline Lent launch_on(Context& ctx, std::size_t n, F body, const After&... after) noexcept {
  return queue(ctx, n, body, after...);
}
template<class T, class Op, class F>
inline Scratch reduce(Context& ctx, T& result, std::size_t n, T identity, Op op, F value) noexcept {
  return reuse::reduce(ctx, result, n, identity, op, value);
}
template<class T, class Op, class F, class... After>
inline Lent reduce_to(Context& ctx, T* out, std::size_t n, T identity, Op op, F value, Scratch* answer,
                      const After&... after) noexcept {
  return reuse::reduce_to(ctx, out, n, identity, op, value, answer, after...);
}
template<class T, class P, class F>
inline Scratch compact(Context& ctx, std::size_t* used, T* out, std::size_t n, P pred, F value) noexcept {
  return reuse::compact(ctx, used, out, n, pred, value);
}

}  // namespace cr::gpu
