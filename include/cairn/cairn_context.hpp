// The execution context device work runs on: where a thread's synchronous work goes, when the host waits for it,
// the streams queued work borrows, and the scratch arena reductions and scans draw on. It keeps the semantics CAIRN's
// generated code relies on (src/cairn/runtime/cairn_reuse.hpp:1-267, cairn_exec.hpp:25-67):
//
//  - Synchronous work returns once the stream it ran on has finished it, and waits for nothing else (never the whole
//    device). It runs on the context's home stream, made by the first work that needs it, or on a stream the caller
//    bound, after what the caller queued there.
//  - A held run queues its synchronous work and waits once: when the outermost run settles, or earlier where the host
//    is about to observe device memory (observed()). An enqueued call queues on the caller's stream and never waits,
//    makes nothing and allocates nothing, so a caller may capture it in a graph.
//  - Queued work borrows a stream of its own (a ticket) until its one wait; a ticket taken while a run is held or a
//    stream is bound starts after what was queued there.
//  - The arena is handed from one user to the next in stream order, by an event, never by stopping the host. A
//    budget reserves it up front and may let it grow to a stated limit; past the limit a request is answered
//    over_budget and nothing changes. Growth is the one step that may stop the host, and only when allocation is
//    synchronous.
//
// The context is written once against a machine M (the HIP machine of cairn_hip.hpp, the host machine of
// cairn_emulate.hpp, or a test's recorder), which supplies:
//
//   Stream, Event                         handles
//   open_stream(), close_stream(s)        a stream at the default priority; its release
//   open_event(), close_event(e)
//   mark(e, s)                            e completes once what is queued on s so far has run
//   after(s, e)                           what is queued on s from now on starts after e
//   drain(s), drain_event(e)              the host waits for s, or for e
//   take(bytes), give(p)                  device memory at once, and its release
//   take_async(bytes, s), give_async(p, s)  the same ordered on s
//   copy(dst, src, bytes, Dir, s)         a copy queued on s
//   fold / scan / lanes                   the device algorithms the operations below queue (cairn_hip_kernels.hpp)
//
// A broken rule (a ticket dropped unawaited, a context destroyed with work open, a wait inside an enqueued call, an
// arena leased twice) is a bug in the caller, and traps.
#pragma once
#include <cstddef>
#include <cstdint>
#include <limits>
#include <new>
#include <type_traits>
#include <utility>
#include <vector>
#include "cairn_runtime.hpp"

namespace cr::reuse {

constexpr std::size_t UNBOUNDED = std::numeric_limits<std::size_t>::max();
constexpr unsigned BLOCK = 256;  // a region's default block: four 64-wide waves

// What a context may hold for scratch: `reserve` bytes allocated when it is made (requests within it never
// allocate), growth up to `most` bytes (a limit below the reserve grants the reserve).
struct Budget {
  std::size_t reserve = 0;
  std::size_t most = 0;
};
// How the arena grows: synchronously (the host waits for the arena's last user, then frees and allocates), or in
// stream order (freed and allocated on the requesting stream; the host never waits).
enum class Allocation { synchronous, stream_ordered };
enum class Scratch { ok, over_budget };  // a request for scratch, answered
enum class Where { device, pinned, unified };  // where an owner's storage lives
enum class Dir { h2d, d2h, d2d, h2h };         // which way a copy goes

// The bytes of n elements of T, or a trap where that passes what one allocation can hold.
template<class T> inline std::size_t span(std::size_t n) noexcept {
  if(n > static_cast<std::size_t>(std::numeric_limits<std::ptrdiff_t>::max()) / sizeof(T)) trap();
  return n * sizeof(T);
}

// Consecutive parts of one scratch request, each starting on 256 bytes (what a device allocation guarantees).
class Parts {
  std::size_t used_ = 0;

 public:
  // The offset of a new part of `bytes`.
  std::size_t add(std::size_t bytes) noexcept {
    const std::size_t at = used_;
    if(bytes > UNBOUNDED - 255 || at > UNBOUNDED - 256 - bytes) trap();
    used_ = at + (bytes + 255) / 256 * 256;
    return at;
  }
  std::size_t bytes() const noexcept { return used_ ? used_ : 256; }
};

template<class M> class Context final {
 public:
  using Stream = typename M::Stream;
  using Event = typename M::Event;

  // A stream this context made and an event that marks what was queued on it.
  struct Lane {
    Stream stream{};
    Event marker{};
  };

  explicit Context(M machine = M{}) noexcept : Context(Budget{0, UNBOUNDED}, Allocation::synchronous, std::move(machine)) {}
  explicit Context(Budget budget, Allocation how = Allocation::synchronous, M machine = M{}) noexcept
      : m_(std::move(machine)), arena_(m_, budget, how) {}
  Context(const Context&) = delete;
  Context& operator=(const Context&) = delete;

  // Nothing may still be borrowed or open; the arena's last user has finished before its storage goes. A bound or
  // enqueued stream is the caller's and is never destroyed here.
  ~Context() noexcept {
    if(tickets_ || holds_ || open_) trap();
    arena_.close(m_);
    for(Lane* lane : idle_) {
      shut(*lane);
      delete lane;
    }
    if(home_made_) shut(home_);
    if(caller_marker_made_) m_.close_event(caller_marker_);
  }

  M& machine() noexcept { return m_; }

  // ---- synchronous work

  // The stream a piece of synchronous work queues on; close_sync ends it. Pieces do not nest.
  Stream open_sync() noexcept {
    if(open_) trap();
    open_ = true;
    return route();
  }
  // The end of a piece: the host waits for its stream, except in a held run (which waits later) or an enqueued call
  // (which never does). `seen`: the host reads what it produced, so it is waited for in a held run too.
  void close_sync(bool seen) noexcept {
    if(!open_) trap();
    open_ = false;
    if(mode_ == Mode::enqueued) {
      if(seen) trap();  // nothing waits under an enqueued call
      return;
    }
    if(holds_ && !seen) {
      pending_ = true;
      return;
    }
    m_.drain(route());
    pending_ = false;
  }
  // Before the host observes device memory by other means (an owner's release, a result read back): what a held run
  // queued so far is waited for. Under an enqueued call nothing may wait.
  void observed() noexcept {
    if(mode_ == Mode::enqueued) trap();
    if(pending_) {
      m_.drain(route());
      pending_ = false;
    }
  }

  // A caller's stream for the thread's synchronous work (after what the caller queued there), and back to the
  // context's own. Not while a piece is open, a held run has work pending, or a call is enqueued.
  void bind(Stream s) noexcept {
    rebinding();
    mode_ = Mode::bound;
    caller_ = s;
  }
  void unbind() noexcept {
    rebinding();
    mode_ = Mode::home;
  }

  void hold() noexcept { ++holds_; }
  void settle() noexcept {
    if(!holds_) trap();
    if(--holds_ == 0 && pending_) {
      m_.drain(route());
      pending_ = false;
    }
  }

  // An enqueued call: from here to leave() synchronous work queues on `s` and nothing waits. It starts from a
  // thread holding nothing, and leaving gives the thread back the binding it had.
  void enqueue(Stream s) noexcept {
    if(mode_ == Mode::enqueued || holds_ || open_ || pending_) trap();
    saved_mode_ = mode_;
    saved_caller_ = caller_;
    mode_ = Mode::enqueued;
    caller_ = s;
    holds_ = 1;
  }
  void leave() noexcept {
    if(mode_ != Mode::enqueued || holds_ != 1 || open_) trap();
    holds_ = 0;
    mode_ = saved_mode_;
    caller_ = saved_caller_;
  }

  // ---- queued work

  // A stream for one ticket: an idle one or a new one, never one another ticket holds. While a run is held or a
  // stream is bound, it starts after what was queued there.
  Lane* lend() noexcept {
    Lane* lane;
    if(!idle_.empty()) {
      lane = idle_.back();
      idle_.pop_back();
    } else {
      lane = new(std::nothrow) Lane;
      if(!lane) trap();
      open(*lane);
    }
    ++tickets_;
    if(mode_ != Mode::home || pending_) {
      const Stream from = route();
      const Event e = marker_of_route();
      m_.mark(e, from);
      m_.after(lane->stream, e);
    }
    return lane;
  }
  // A ticket's wait: the host waits for its stream, which then serves the next ticket.
  void take_back(Lane* lane) noexcept {
    if(!tickets_) trap();
    m_.drain(lane->stream);
    --tickets_;
    idle_.push_back(lane);
  }

  // ---- the arena

  // At least `bytes` of scratch for work queued on `s` from now on, ordered after the arena's previous user. Within
  // the capacity nothing is allocated; past the budget's limit the answer is over_budget and nothing changes.
  // unlease(s) must follow once the work that uses it is queued.
  Scratch lease(std::size_t bytes, Stream s, void** out) noexcept { return arena_.lease(m_, bytes, s, out); }
  void unlease(Stream s) noexcept { arena_.unlease(m_, s); }

  // ---- what the tests read

  std::size_t streams_made() const noexcept { return made_; }
  std::size_t tickets() const noexcept { return tickets_; }
  std::size_t capacity() const noexcept { return arena_.size; }
  std::size_t grown() const noexcept { return arena_.regrown; }
  bool bound() const noexcept { return mode_ == Mode::bound; }
  bool enqueued() const noexcept { return mode_ == Mode::enqueued; }

 private:
  enum class Mode : unsigned char { home, bound, enqueued };

  // The arena: one allocation, leased to one user at a time, handed on by the event its last user's stream marked.
  struct Arena {
    Budget budget;
    Allocation how;
    void* base = nullptr;
    std::size_t size = 0, regrown = 0;
    Event fence{};
    bool fence_made = false, fenced = false, leased = false;

    Arena(M& m, Budget b, Allocation h) noexcept : budget(b), how(h) {
      if(budget.most < budget.reserve) budget.most = budget.reserve;
      if(budget.reserve) {
        base = m.take(budget.reserve);
        size = budget.reserve;
      }
    }
    Scratch lease(M& m, std::size_t bytes, Stream s, void** out) noexcept {
      if(leased) trap();
      if(bytes > size) {
        if(bytes > budget.most) return Scratch::over_budget;
        regrow(m, bytes, s);
      }
      if(fenced) m.after(s, fence);
      *out = base;
      leased = true;
      return Scratch::ok;
    }
    void unlease(M& m, Stream s) noexcept {
      if(!leased) trap();
      if(!fence_made) {
        fence = m.open_event();
        fence_made = true;
      }
      m.mark(fence, s);
      fenced = true;
      leased = false;
    }
    void regrow(M& m, std::size_t bytes, Stream s) noexcept {
      if(how == Allocation::stream_ordered) {
        if(base) {
          if(fenced) m.after(s, fence);
          m.give_async(base, s);
        }
        base = m.take_async(bytes, s);
      } else {
        if(base) {
          if(fenced) m.drain_event(fence);
          m.give(base);
        }
        base = m.take(bytes);
      }
      fenced = false;  // nothing queued reaches the new storage yet (in stream order, s already waited)
      size = bytes;
      ++regrown;
    }
    void close(M& m) noexcept {
      if(leased) trap();
      if(fenced) m.drain_event(fence);
      if(base) m.give(base);
      if(fence_made) m.close_event(fence);
    }
  };

  void open(Lane& lane) noexcept {
    lane.stream = m_.open_stream();
    lane.marker = m_.open_event();
    ++made_;
  }
  void shut(Lane& lane) noexcept {
    m_.close_event(lane.marker);
    m_.close_stream(lane.stream);
  }
  Stream route() noexcept {
    if(mode_ != Mode::home) return caller_;
    if(!home_made_) {
      open(home_);
      home_made_ = true;
    }
    return home_.stream;
  }
  Event marker_of_route() noexcept {
    if(mode_ == Mode::home) return home_.marker;  // route() made it
    if(!caller_marker_made_) {
      caller_marker_ = m_.open_event();
      caller_marker_made_ = true;
    }
    return caller_marker_;
  }
  void rebinding() noexcept {
    if(open_ || pending_ || mode_ == Mode::enqueued) trap();
  }

  M m_;
  Arena arena_;
  Lane home_{};
  bool home_made_ = false;
  std::vector<Lane*> idle_;
  std::size_t tickets_ = 0, made_ = 0;
  Mode mode_ = Mode::home, saved_mode_ = Mode::home;
  Stream caller_{}, saved_caller_{};
  Event caller_marker_{};
  bool caller_marker_made_ = false;
  unsigned holds_ = 0;
  bool pending_ = false, open_ = false;
};

// Queued work's ticket: a stream of the context's, held until the ticket's one wait, which hands it back once its
// work has run. Move-only; dropping one unawaited traps.
template<class M> class Lent final {
  Context<M>* ctx_;
  typename Context<M>::Lane* lane_;

 public:
  explicit Lent(Context<M>& ctx) noexcept : ctx_(&ctx), lane_(ctx.lend()) {}
  Lent(Lent&& o) noexcept : ctx_(o.ctx_), lane_(std::exchange(o.lane_, nullptr)) {}
  Lent(const Lent&) = delete;
  Lent& operator=(const Lent&) = delete;
  Lent& operator=(Lent&&) = delete;
  ~Lent() noexcept {
    if(lane_) trap();
  }
  typename M::Stream stream() const noexcept { return lane_->stream; }
  // An event that completes with what is queued on the ticket's stream so far, and ordering after one.
  typename M::Event mark() const noexcept {
    ctx_->machine().mark(lane_->marker, lane_->stream);
    return lane_->marker;
  }
  void follow(typename M::Event e) const noexcept { ctx_->machine().after(lane_->stream, e); }
  void wait() && noexcept { ctx_->take_back(std::exchange(lane_, nullptr)); }
};

// A piece of synchronous work as a scope: stream() is where it queues; the scope's end closes it (a wait, unless
// held or enqueued). `seen`: the host reads what it produced, so what a held run queued before is waited for first
// and the piece itself is waited for, held or not.
template<class M> class Sync final {
  Context<M>& ctx_;
  bool seen_;
  typename M::Stream s_;

 public:
  explicit Sync(Context<M>& ctx, bool seen = false) noexcept : ctx_(ctx), seen_(seen) {
    if(seen) ctx.observed();
    s_ = ctx.open_sync();
  }
  ~Sync() noexcept { ctx_.close_sync(seen_); }
  Sync(const Sync&) = delete;
  Sync& operator=(const Sync&) = delete;
  typename M::Stream stream() const noexcept { return s_; }
};

// Scratch from the context's arena as a scope, for work queued on one stream: handed on (its fence marked on that
// stream) when the scope ends.
template<class M> class Lease final {
  Context<M>& ctx_;
  typename M::Stream s_;
  char* base_ = nullptr;
  Scratch answer_;

 public:
  Lease(Context<M>& ctx, typename M::Stream s, std::size_t bytes) noexcept : ctx_(ctx), s_(s) {
    void* p = nullptr;
    answer_ = ctx.lease(bytes, s, &p);
    base_ = static_cast<char*>(p);
  }
  ~Lease() noexcept {
    if(answer_ == Scratch::ok) ctx_.unlease(s_);
  }
  Lease(const Lease&) = delete;
  Lease& operator=(const Lease&) = delete;
  Scratch answer() const noexcept { return answer_; }
  explicit operator bool() const noexcept { return answer_ == Scratch::ok; }
  template<class T> T* at(std::size_t offset) const noexcept { return reinterpret_cast<T*>(base_ + offset); }
};

// Synchronous work: `queue(stream)` queues it; the call returns once it has run (at once in a held run or an enqueued
// call). What emitted device code runs through (src/cairn/compiler/device/launches.py:65).
template<class M, class Q> inline void synchronous(Context<M>& ctx, Q&& queue) noexcept {
  const Sync<M> on(ctx);
  queue(on.stream());
}
// The same for work whose result the host reads when the call returns (a copy to host memory): waited for always.
template<class M, class Q> inline void observed(Context<M>& ctx, Q&& queue) noexcept {
  const Sync<M> on(ctx, true);
  queue(on.stream());
}

// A value as an element of type R: the identity conversion, or one a type that checks itself declares.
template<class R, class T> CR_HD inline R landed(const T& x) noexcept { return static_cast<R>(x); }

// The total a fold left in scratch, stored as the element type of its destination.
template<class R, class T> struct Landing {
  R* at;
  const T* total;
  CR_HD void operator()(std::size_t) const noexcept { *at = landed<R>(*total); }
};

// out[i] from the inclusive scan h: h[i], or (exclusive) h[i - 1] with the identity first.
template<bool Exclusive, class R, class T> struct Shifted {
  R* out;
  const T* h;
  T identity;
  CR_HD void operator()(std::size_t i) const noexcept {
    out[i] = landed<R>(Exclusive ? (i ? h[i - 1] : identity) : h[i]);
  }
};

// The folds, scans and compaction on the arena. The machine computes each in a fixed association for a given n
// (fold_space / scan_space tell how much scratch it needs), so two runs give the same bits; the operator must be
// associative and commutative, which the integer and min/max folds the language admits here are, and a float sum's
// result lies within its usual bound in any order.

// The fold of value(i) over i < n from `identity`, read back to the host into `result`. Over budget nothing is queued
// and `result` keeps its value.
template<class M, class T, class Op, class F>
inline Scratch reduce(Context<M>& ctx, T& result, std::size_t n, T identity, Op op, F value) noexcept {
  if(!n) {
    result = identity;
    return Scratch::ok;
  }
  Parts parts;
  const std::size_t cell = parts.add(sizeof(T)), work = parts.add(M::template fold_space<T>(n));
  T got = identity;
  Scratch answer;
  {
    const Sync<M> on(ctx, true);
    const Lease<M> lease(ctx, on.stream(), parts.bytes());
    answer = lease.answer();
    if(lease) {
      M& m = ctx.machine();
      m.fold(n, value, op, identity, lease.template at<T>(cell), lease.template at<void>(work), on.stream());
      m.copy(&got, lease.template at<T>(cell), sizeof(T), Dir::d2h, on.stream());
    }
  }
  if(answer == Scratch::ok) result = got;
  return answer;
}

// The fold into `out`, a device cell, on a ticket of its own queued after the tickets `after...`; the total stays on
// the device for work ordered after the returned ticket. Over budget nothing but the ordering is queued.
template<class M, class T, class Op, class F, class... After>
inline Lent<M> reduce_to(Context<M>& ctx, T* out, std::size_t n, T identity, Op op, F value, Scratch* answer,
                         const After&... after) noexcept {
  ctx.observed();
  Lent<M> t(ctx);
  (t.follow(after.mark()), ...);
  Parts parts;
  const std::size_t work = parts.add(M::template fold_space<T>(n));
  const Lease<M> lease(ctx, t.stream(), parts.bytes());
  *answer = lease.answer();
  if(lease) ctx.machine().fold(n, value, op, identity, out, lease.template at<void>(work), t.stream());
  return t;
}

// The fold with its total stored at `at`, a device element, as synchronous work: nothing crosses to the host, and in
// a held run nothing waits.
template<class M, class T, class R, class Op, class F>
inline Scratch reduce_into(Context<M>& ctx, R* at, std::size_t n, T identity, Op op, F value) noexcept {
  const Sync<M> on(ctx);
  Parts parts;
  const std::size_t cell = std::is_same_v<R, T> ? 0 : parts.add(sizeof(T));
  const std::size_t work = parts.add(M::template fold_space<T>(n));
  const Lease<M> lease(ctx, on.stream(), parts.bytes());
  if(!lease) return lease.answer();
  M& m = ctx.machine();
  if constexpr(std::is_same_v<R, T>) {
    m.fold(n, value, op, identity, at, lease.template at<void>(work), on.stream());
  } else {
    T* total = lease.template at<T>(cell);
    m.fold(n, value, op, identity, total, lease.template at<void>(work), on.stream());
    m.template lanes<1>(1, Landing<R, T>{at, total}, on.stream(), 64, 1);
  }
  return Scratch::ok;
}

// The scan of value(i) into out (inclusive, or exclusive when Exclusive), queued on `s`: the inclusive scan lands in
// the arena first, so a value(i) that reads out[j] reads it before anything writes it; then out from there, and with
// `last` the total's copy to the host (the caller's wait completes it).
template<bool Exclusive, class M, class T, class R, class Op, class F>
inline Scratch scanned(Context<M>& ctx, typename M::Stream s, T* last, R* out, std::size_t n, T identity, Op op,
                       F value) noexcept {
  Parts parts;
  const std::size_t held = parts.add(span<T>(n)), work = parts.add(M::template scan_space<T>(n));
  const Lease<M> lease(ctx, s, parts.bytes());
  if(!lease) return lease.answer();
  M& m = ctx.machine();
  T* h = lease.template at<T>(held);
  m.scan(n, value, op, identity, h, lease.template at<void>(work), s);
  m.template lanes<1>(n, Shifted<Exclusive, R, T>{out, h, identity}, s, BLOCK, 4);
  if(last) m.copy(last, h + (n - 1), sizeof(T), Dir::d2h, s);
  return Scratch::ok;
}

// The scan with its total for the host (op over every value), waited for.
template<bool Exclusive, class M, class T, class R, class Op, class F>
inline Scratch scan(Context<M>& ctx, T& total, R* out, std::size_t n, T identity, Op op, F value) noexcept {
  if(!n) {
    total = identity;
    return Scratch::ok;
  }
  T got = identity;
  Scratch answer;
  {
    const Sync<M> on(ctx, true);
    answer = scanned<Exclusive>(ctx, on.stream(), &got, out, n, identity, op, value);
  }
  if(answer == Scratch::ok) total = got;
  return answer;
}

// The scan with no total for the host: synchronous work, which in a held run waits for nothing.
template<bool Exclusive, class M, class T, class R, class Op, class F>
inline Scratch scan_into(Context<M>& ctx, R* out, std::size_t n, T identity, Op op, F value) noexcept {
  if(!n) return Scratch::ok;
  const Sync<M> on(ctx);
  return scanned<Exclusive>(ctx, on.stream(), static_cast<T*>(nullptr), out, n, identity, op, value);
}

// Compaction's three steps: each index's selection kept once, its inclusive count of selections, and the selected
// values written at their count's place.
template<class P> struct Select {
  P pred;
  unsigned char* keep;
  CR_HD void operator()(std::size_t i) const noexcept { keep[i] = pred(i) ? 1 : 0; }
};
struct Kept {
  const unsigned char* keep;
  CR_HD std::size_t operator()(std::size_t i) const noexcept { return keep[i]; }
};
struct Plus {
  CR_HD std::size_t operator()(std::size_t a, std::size_t b) const noexcept { return a + b; }
};
template<class T, class F> struct Place {
  F value;
  const unsigned char* keep;
  const std::size_t* count;
  T* out;
  CR_HD void operator()(std::size_t i) const noexcept {
    if(keep[i]) out[count[i] - 1] = value(i);
  }
};

// Stable compaction: value(i) for each i with pred(i), in order, into the front of out (the rest of out is left as
// it was); pred runs exactly once an index, value only where selected. `*used` is the count selected (0 over budget).
template<class M, class T, class P, class F>
inline Scratch compact(Context<M>& ctx, std::size_t* used, T* out, std::size_t n, P pred, F value) noexcept {
  *used = 0;
  if(!n) return Scratch::ok;
  Parts parts;
  const std::size_t flags = parts.add(n), counts = parts.add(span<std::size_t>(n));
  const std::size_t work = parts.add(M::template scan_space<std::size_t>(n));
  std::size_t total = 0;
  Scratch answer;
  {
    const Sync<M> on(ctx, true);
    const Lease<M> lease(ctx, on.stream(), parts.bytes());
    answer = lease.answer();
    if(lease) {
      M& m = ctx.machine();
      unsigned char* keep = lease.template at<unsigned char>(flags);
      std::size_t* count = lease.template at<std::size_t>(counts);
      m.template lanes<1>(n, Select<P>{pred, keep}, on.stream(), BLOCK, 4);
      m.scan(n, Kept{keep}, Plus{}, std::size_t(0), count, lease.template at<void>(work), on.stream());
      m.template lanes<1>(n, Place<T, F>{value, keep, count, out}, on.stream(), BLOCK, 4);
      m.copy(&total, count + (n - 1), sizeof(total), Dir::d2h, on.stream());
    }
  }
  if(answer == Scratch::ok) *used = total;
  return answer;
}

}  // namespace cr::reuse
