// The operations generated device code calls on the thread's execution context, written once for whichever machine
// cr::gpu::Machine names. The spellings and what each one waits for are CAIRN's (src/cairn/runtime/cairn_exec.hpp:
// 68-230; the lowering that emits them: src/cairn/compiler/lower/execution.py, plans/chunks.py, plans/staging.py,
// primitives/builtins.py:280): scoped owners, `run` and its vector and staged plans, `transfer`, reductions, scans and
// compaction on the context's arena, and queued work on tickets.
#pragma once
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <type_traits>
#include <utility>
#include "cairn_here.hpp"

namespace cr::gpu {

// Scoped owners of zero-initialized storage: released at scope exit, never copied or moved; n of 0 owns nothing.
// Device and unified storage is zeroed as synchronous work the host waits for, so later work on any stream sees
// zeros; pinned storage is host memory, zeroed on the host. What a held run queued is waited for before the storage
// is taken or given back.
template<class T, Where W> class Owner final {
  T* data_ = nullptr;

 public:
  explicit Owner(std::size_t n) noexcept {
    static_assert(std::is_trivially_copyable_v<T>, "zeroed bytes are a value of T");
    const std::size_t bytes = reuse::span<T>(n);
    if(!bytes) return;
    Context& ctx = here();
    ctx.observed();
    data_ = static_cast<T*>(ctx.machine().take_where(W, bytes));
    if constexpr(W == Where::pinned) {
      std::memset(static_cast<void*>(data_), 0, bytes);
    } else {
      const reuse::Sync<Machine> on(ctx, true);
      ctx.machine().zero(data_, bytes, on.stream());
    }
  }
  ~Owner() noexcept {
    if(!data_) return;
    Context& ctx = here();
    ctx.observed();
    ctx.machine().give_where(W, data_);
  }
  Owner(const Owner&) = delete;
  Owner& operator=(const Owner&) = delete;
  T* data() const noexcept { return data_; }
};
template<class T> using Buffer = Owner<T, Where::device>;
template<class T> using Pinned = Owner<T, Where::pinned>;
template<class T> using Unified = Owner<T, Where::unified>;

// `parallel i in n`: body(i) once for every i below n, as synchronous work. `block` threads a block and about
// `per_lane` indices a thread are a plan's choice; the indices run are the same whatever it chose.
template<unsigned U = 1, class F>
inline void run(Context& ctx, std::size_t n, F body, unsigned block = reuse::BLOCK, std::size_t per_lane = 1) noexcept {
  static_assert(std::is_trivially_copyable_v<F>, "a lane body crosses over as kernel arguments");
  if(!n) return;
  const reuse::Sync<Machine> on(ctx);
  ctx.machine().template lanes<U>(n, body, on.stream(), block, per_lane);
}

// `plan vector W`: a W-wide chunk of each array a lane touches only at [i], one aligned access each. `whole` (every
// chunked pointer on its chunk's width, aligned<W>(...)) decides for the region; otherwise the scalar lanes run.
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
  const reuse::Sync<Machine> on(ctx);
  ctx.machine().template vector_lanes<W, U>(n, scalar, chunk, on.stream(), block, per_lane);
}

// `plan stage R`: a block's tiles of its width with R halo elements a side in LDS; bytes(width) is what the staged
// arrays of a tile of `width` elements take, each array starting on 16 bytes.
template<class T> CR_HD constexpr std::size_t tile_bytes(std::size_t width) noexcept {
  return (width * sizeof(T) + 15) / 16 * 16;
}
template<std::size_t R, unsigned U = 1, class L, class F, class S>
inline void run_staged(Context& ctx, std::size_t n, L load, F body, S bytes, unsigned block = reuse::BLOCK,
                       std::size_t per_lane = 1) noexcept {
  static_assert(std::is_trivially_copyable_v<L> && std::is_trivially_copyable_v<F>, "lanes cross as arguments");
  if(!n) return;
  const reuse::Sync<Machine> on(ctx);
  ctx.machine().template staged_lanes<R, U>(n, load, body, bytes, on.stream(), block, per_lane);
}

// `transfer(dst, src)`: n elements. Between device views it is device work like a region; to or from host memory the
// host waits for it, held or not (the host may read or change its side as soon as the call returns).
template<class T> inline void copy_on(Context& ctx, T* dst, const T* src, std::size_t n, Dir d) noexcept {
  if(!n) return;
  const reuse::Sync<Machine> on(ctx, d != Dir::d2d);
  ctx.machine().copy(dst, src, reuse::span<T>(n), d, on.stream());
}

// Reductions, scans and compaction on the thread's context, whose budget has no limit: over_budget would be a
// failed allocation, and traps like one.
inline void granted(Scratch answer) noexcept {
  if(answer != Scratch::ok) trap();
}
template<class T, class Op, class F> inline T reduce_on(Context& ctx, std::size_t n, T identity, Op op, F value) noexcept {
  T result = identity;
  granted(reuse::reduce(ctx, result, n, identity, op, value));
  return result;
}
template<bool Exclusive, class T, class R, class Op, class F>
inline T scan_on(Context& ctx, R* out, std::size_t n, T identity, Op op, F value) noexcept {
  T total = identity;
  granted(reuse::scan<Exclusive>(ctx, total, out, n, identity, op, value));
  return total;
}
template<class T, class R, class Op, class F>
inline void reduce_into(Context& ctx, R* at, std::size_t n, T identity, Op op, F value) noexcept {
  granted(reuse::reduce_into(ctx, at, n, identity, op, value));
}
template<bool Exclusive, class T, class R, class Op, class F>
inline void scan_into(Context& ctx, R* out, std::size_t n, T identity, Op op, F value) noexcept {
  granted(reuse::scan_into<Exclusive>(ctx, out, n, identity, op, value));
}
template<class T, class P, class F>
inline std::size_t compact_on(Context& ctx, T* out, std::size_t n, P pred, F value) noexcept {
  std::size_t used = 0;
  granted(reuse::compact(ctx, &used, out, n, pred, value));
  return used;
}

// Queued work (`spawn parallel ... after t`, `spawn transfer`): on a ticket of its own, after the tickets `after...`,
// returned at once; its wait is the host's, so a held run's work is waited for first.
template<class F, class... After> inline Lent queue(Context& ctx, std::size_t n, F body, const After&... after) noexcept {
  static_assert(std::is_trivially_copyable_v<F>, "a lane body crosses over as kernel arguments");
  ctx.observed();
  Lent t(ctx);
  (t.follow(after.mark()), ...);
  if(n) ctx.machine().template lanes<1>(n, body, t.stream(), reuse::BLOCK, 1);
  return t;
}
template<class T, class... After>
inline Lent queue_copy(Context& ctx, T* dst, const T* src, std::size_t n, Dir d, const After&... after) noexcept {
  ctx.observed();
  Lent t(ctx);
  (t.follow(after.mark()), ...);
  if(n) ctx.machine().copy(dst, src, reuse::span<T>(n), d, t.stream());
  return t;
}
inline void wait(Lent&& t) noexcept { std::move(t).wait(); }

// The same operations for a program or a test holding a context of its own, with a budget it declared.
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
