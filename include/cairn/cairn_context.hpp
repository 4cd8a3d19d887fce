// The execution context device work runs through, written against a machine (a template parameter): the HIP machine
// of cairn_hip.hpp on a GPU, a recording host machine in the tests. It keeps the semantics CAIRN-emitted code relies
// on (src/cairn/runtime/cairn_reuse.hpp:1-525, cairn_exec.hpp:1-230):
//
//  - synchronous work runs on one lane (a stream and an event) and the call returns once that stream has run it,
//    never by waiting for the whole device;
//  - a caller may bind its own stream: synchronous work then runs there, after what the caller queued;
//  - a held run queues all its synchronous work on one lane and waits once, at its end;
//  - an enqueued call queues on the caller's stream and never waits;
//  - lanes are made on first use and kept: work repeated on a thread makes no stream and allocates nothing;
//  - scratch comes from one arena whose size the context declares when it is made (a budget: a reserve allocated up
//    front, a limit it may grow to). The arena passes from one user to the next in stream order, through an event
//    the next user's stream waits on, so the host never stops for it; a request past the limit is answered
//    over_budget and changes nothing;
//  - queued work borrows a lane as a Lent ticket, which exactly one wait hands back.
//
// Misuse (a lane never given back, nested synchronous work on a bound stream, a wait inside an enqueued call, the
// arena leased twice, a ticket dropped unawaited) traps.
//
// The operations below (reduce, scan, compact) are written once against the machine's primitives: `lanes` runs a
// body for every index of a range, `reduce`, `inclusive_scan` and `exclusive_sum` are the device library's (asked
// first, with no storage, how much temporary storage they need), `copy` moves bytes on a stream.
#pragma once
#include <cstddef>
#include <cstdint>
#include <iterator>
#include <limits>
#include <new>
#include <utility>
#include "cairn_runtime.hpp"

// A lane body's marker: device code under hipcc, a plain lambda on the host machine of the tests.
#if defined(__HIPCC__)
#define CR_DEVICE __device__
#else
#define CR_DEVICE
#endif

namespace cr::reuse {

constexpr unsigned BLOCK = 256;      // threads a lane launch's block holds unless a plan says otherwise: 4 waves
constexpr std::size_t ALIGN = 256;   // the alignment hipMalloc gives and scratch carved from the arena keeps
constexpr std::size_t UNBOUNDED = std::numeric_limits<std::size_t>::max();

// The scratch a context may hold: `reserve` bytes allocated when it is made (a request within them never allocates),
// growth up to `most` (a limit below the reserve grants nothing more).
struct Budget {
  std::size_t reserve = 0;
  std::size_t most = 0;
};
// How the arena's storage is taken and given back when it grows: at once (the one place a context may wait for the
// device), or ordered on the stream of the work that needs it.
enum class Allocation { synchronous, stream_ordered };
enum class Scratch { ok, over_budget };        // what a request for scratch was answered
enum class Where { device, pinned, unified };  // where an owner's storage lives
enum class Dir { h2d, d2h, d2d, h2h };         // which way a copy crosses

// The bytes of n elements of T, or a trap where they would not fit a ptrdiff_t.
template<class T> inline std::size_t span(std::size_t n) noexcept {
  if(n > static_cast<std::size_t>(std::numeric_limits<std::ptrdiff_t>::max()) / sizeof(T)) trap();
  return n * sizeof(T);
}
// b rounded up to ALIGN, or a trap where that overflows.
inline std::size_t aligned(std::size_t b) noexcept {
  if(b > UNBOUNDED - ALIGN) trap();
  return (b + ALIGN - 1) & ~(ALIGN - 1);
}

template<class Api> class Context final {
public:
  using Stream = typename Api::Stream;
  using Event = typename Api::Event;
  struct Lane {
    Stream stream{};
    Event event{};
    Lane* next = nullptr;  // the free list
  };

  // A context with no scratch until asked for, then as much as asked: the thread context's budget.
  explicit Context(Api api = Api{}) noexcept : Context(Budget{0, UNBOUNDED}, Allocation::synchronous, std::move(api)) {}
  explicit Context(Budget budget, Allocation how = Allocation::synchronous, Api api = Api{}) noexcept
      : api_(std::move(api)), budget_(budget), how_(how) {
    if(budget_.most < budget_.reserve) budget_.most = budget_.reserve;
    if(budget_.reserve) {
      arena_ = api_.alloc(budget_.reserve);
      capacity_ = budget_.reserve;
    }
  }
  Context(const Context&) = delete;
  Context& operator=(const Context&) = delete;
  ~Context() noexcept {
    if(lent_ || held_ || holding_ || leased_) trap();  // work nobody waited for, or scratch never given back
    if(used_) api_.sync_event(marker_);                 // the arena's last user has finished before it goes
    if(arena_) api_.free(arena_);
    while(free_) {
      Lane* lane = free_;
      free_ = lane->next;
      api_.destroy_event(lane->event);
      api_.destroy_stream(lane->stream);
      delete lane;
    }
    if(bound_event_) api_.destroy_event(bound_.event);
    if(marked_) api_.destroy_event(marker_);
  }

  // A lane for work about to be queued: for synchronous work the held run's lane, else the bound stream, else a
  // free lane (made if none). Another lane lent while a run is held or a stream bound starts after that work.
  Lane* lend(bool synchronous = false) noexcept {
    if(synchronous && held_) return held_;
    if(synchronous && binding_) {
      if(bound_lent_) trap();
      bound_lent_ = true;
      ++lent_;
      return &bound_;
    }
    Lane* lane = free_;
    if(lane) free_ = lane->next;
    else {
      lane = new(std::nothrow) Lane;
      if(!lane) trap();
      lane->stream = api_.make_stream();
      lane->event = api_.make_event();
      ++made_;
    }
    lane->next = nullptr;
    ++lent_;
    if(held_ || binding_) {
      Lane& before = held_ ? *held_ : bound_;
      api_.record(event_of(before), before.stream);
      api_.wait_event(lane->stream, before.event);
    }
    return lane;
  }
  // Wait for the lane's work (not under an enqueued call, whose stream the caller synchronizes) and keep the lane.
  void give_back(Lane* lane) noexcept {
    if(lane == held_) held_ = nullptr;
    if(!(enqueued_ && lane == &bound_)) api_.sync_stream(lane->stream);
    --lent_;
    if(lane == &bound_) {
      bound_lent_ = false;
      return;
    }
    lane->next = free_;
    free_ = lane;
  }
  // The end of synchronous work: wait now, or in a held run at its end.
  void finish(Lane* lane) noexcept {
    if(holding_) held_ = lane;
    else give_back(lane);
  }

  void bind(Stream stream) noexcept {
    if(bound_lent_ || enqueued_) trap();
    bound_.stream = stream;
    binding_ = true;
  }
  void unbind() noexcept {
    if(bound_lent_ || enqueued_) trap();
    binding_ = false;
  }
  void hold() noexcept { ++holding_; }
  void settle() noexcept {
    if(!holding_) trap();
    if(--holding_ == 0 && held_) give_back(held_);
  }
  void enqueue(Stream stream) noexcept {
    if(enqueued_ || holding_ || bound_lent_) trap();
    saved_binding_ = binding_;
    saved_stream_ = bound_.stream;
    bound_.stream = stream;
    binding_ = enqueued_ = true;
    holding_ = 1;
  }
  void leave() noexcept {
    if(!enqueued_ || holding_ != 1) trap();
    if(held_) give_back(held_);
    holding_ = 0;
    enqueued_ = false;
    binding_ = saved_binding_;
    bound_.stream = saved_stream_;
  }
  // Before the host reads a result: wait for the held run so far. An enqueued call never waits.
  void observed() noexcept {
    if(enqueued_) trap();
    if(held_) give_back(held_);
  }

  // Scratch of at least `bytes` for work about to be queued on `lane`, ordered after the arena's previous user (the
  // lane's stream waits on the event that user's release recorded); the host does not wait. Within the capacity
  // nothing is allocated; past it the arena grows up to the budget's limit; past the limit the answer is
  // over_budget and nothing changes. release(lane) follows once the work using it is queued.
  Scratch acquire(std::size_t bytes, Lane& lane, void** out) noexcept {
    if(leased_) trap();
    if(bytes > capacity_) {
      if(bytes > budget_.most) return Scratch::over_budget;
      grow(bytes, lane);
    }
    if(!marked_) {
      marker_ = api_.make_event();
      marked_ = true;
    }
    if(used_) api_.wait_event(lane.stream, marker_);
    *out = arena_;
    leased_ = true;
    return Scratch::ok;
  }
  // The arena's user is queued on `lane`: the next one waits for what was queued there so far.
  void release(Lane& lane) noexcept {
    if(!leased_) trap();
    api_.record(marker_, lane.stream);
    used_ = true;
    leased_ = false;
  }

  std::size_t capacity() const noexcept { return capacity_; }
  std::size_t grown() const noexcept { return grown_; }
  std::size_t streams_made() const noexcept { return made_; }
  std::size_t lent() const noexcept { return lent_; }
  bool bound() const noexcept { return binding_; }
  bool enqueued() const noexcept { return enqueued_; }
  Api& api() noexcept { return api_; }

private:
  Event event_of(Lane& lane) noexcept {
    if(&lane == &bound_ && !bound_event_) bound_.event = api_.make_event(), bound_event_ = true;
    return lane.event;
  }
  // A larger arena. Stream-ordered: the old storage is freed on `lane`'s stream once the previous user is done (the
  // stream waits on the marker first), the new one taken there. Synchronous: the host waits for the previous user,
  // frees, and allocates; no queued work can reach the new storage yet.
  void grow(std::size_t bytes, Lane& lane) noexcept {
    void* old = arena_;
    arena_ = nullptr;
    if(how_ == Allocation::stream_ordered) {
      if(old) {
        if(used_) api_.wait_event(lane.stream, marker_);
        api_.free_async(old, lane.stream);
      }
      arena_ = api_.alloc_async(bytes, lane.stream);
    } else {
      if(old) {
        if(used_) api_.sync_event(marker_);
        api_.free(old);
      }
      arena_ = api_.alloc(bytes);
      used_ = false;
    }
    capacity_ = bytes;
    ++grown_;
  }

  Api api_;
  Budget budget_;
  Allocation how_;
  Lane* free_ = nullptr;
  std::size_t lent_ = 0, made_ = 0, holding_ = 0, grown_ = 0;
  Lane bound_{};
  bool binding_ = false, bound_lent_ = false, bound_event_ = false, enqueued_ = false;
  Lane* held_ = nullptr;
  bool saved_binding_ = false;
  Stream saved_stream_{};
  void* arena_ = nullptr;
  std::size_t capacity_ = 0;
  Event marker_{};       // recorded where the arena's last user was queued
  bool marked_ = false;  // marker_ made
  bool used_ = false;    // marker_ recorded since the arena last changed
  bool leased_ = false;  // between acquire and release
};

// Work queued on a lane the context lent, as a ticket: exactly one wait() hands the lane back once its work is done;
// a ticket dropped unawaited traps. mark() gives an event later work can be ordered after, follow() orders this
// lane after another's.
template<class Api> class Lent final {
  using Lane = typename Context<Api>::Lane;
  Context<Api>* ctx_;
  Lane* lane_;

public:
  explicit Lent(Context<Api>& ctx) noexcept : ctx_(&ctx), lane_(ctx.lend()) {}
  Lent(Lent&& other) noexcept : ctx_(other.ctx_), lane_(std::exchange(other.lane_, nullptr)) {}
  Lent(const Lent&) = delete;
  Lent& operator=(const Lent&) = delete;
  Lent& operator=(Lent&&) = delete;
  ~Lent() noexcept {
    if(lane_) trap();
  }
  typename Api::Stream stream() const noexcept { return lane_->stream; }
  Lane& lane() const noexcept { return *lane_; }
  typename Api::Event mark() const noexcept {
    ctx_->api().record(lane_->event, lane_->stream);
    return lane_->event;
  }
  void follow(typename Api::Event e) const noexcept { ctx_->api().wait_event(lane_->stream, e); }
  void wait() && noexcept { ctx_->give_back(std::exchange(lane_, nullptr)); }
};

// Synchronous work: queued on the context's synchronous lane; returns once that lane has run it (at once in a held
// run, whose end waits).
template<class Api, class Q> inline void synchronous(Context<Api>& ctx, Q&& queue) noexcept {
  typename Context<Api>::Lane* lane = ctx.lend(true);
  queue(lane->stream);
  ctx.finish(lane);
}
// Work whose result the host reads on return (a copy to host memory): it waits, in a held run too, and traps under
// an enqueued call.
template<class Api, class Q> inline void observed(Context<Api>& ctx, Q&& queue) noexcept {
  ctx.observed();
  typename Context<Api>::Lane* lane = ctx.lend(true);
  queue(lane->stream);
  ctx.give_back(lane);
}

// The combining operator with its value type named, for the device library's dispatch.
template<class T, class Op> struct Binary {
  Op op;
  CR_HD T operator()(const T& a, const T& b) const { return op(a, b); }
};
// A random-access input iterator whose element i is value(i).
template<class T, class F> struct Indexed {
  using value_type = T;
  using reference = T;
  using pointer = void;
  using difference_type = std::ptrdiff_t;
  using iterator_category = std::random_access_iterator_tag;
  F value;
  std::size_t i = 0;
  CR_HD T operator*() const { return value(i); }
  CR_HD T operator[](difference_type d) const { return value(i + static_cast<std::size_t>(d)); }
  CR_HD Indexed operator+(difference_type d) const { return Indexed{value, i + static_cast<std::size_t>(d)}; }
  CR_HD Indexed operator-(difference_type d) const { return Indexed{value, i - static_cast<std::size_t>(d)}; }
  CR_HD difference_type operator-(const Indexed& o) const { return difference_type(i) - difference_type(o.i); }
  CR_HD Indexed& operator+=(difference_type d) {
    i += static_cast<std::size_t>(d);
    return *this;
  }
  CR_HD Indexed& operator-=(difference_type d) {
    i -= static_cast<std::size_t>(d);
    return *this;
  }
  CR_HD Indexed& operator++() {
    ++i;
    return *this;
  }
  CR_HD Indexed operator++(int) {
    Indexed before = *this;
    ++i;
    return before;
  }
  CR_HD Indexed& operator--() {
    --i;
    return *this;
  }
  CR_HD bool operator==(const Indexed& o) const { return i == o.i; }
  CR_HD bool operator!=(const Indexed& o) const { return i != o.i; }
  CR_HD bool operator<(const Indexed& o) const { return i < o.i; }
};

// value(i) folded with op over [0, n), identity for n = 0, its result on the host: the total lands in one cell of
// the arena, then one copy and one wait bring it back. The association order is the device library's. Over the
// budget nothing is queued and `result` is left alone.
template<class Api, class T, class Op, class F>
inline Scratch reduce(Context<Api>& ctx, T& result, std::size_t n, T identity, Op op, F value) noexcept {
  if(!n) {
    result = identity;
    return Scratch::ok;
  }
  ctx.observed();
  Api& api = ctx.api();
  auto* lane = ctx.lend(true);
  const Indexed<T, F> in{value};
  const Binary<T, Op> fold{op};
  std::size_t need = 0;
  api.reduce(nullptr, need, in, static_cast<T*>(nullptr), n, fold, identity, lane->stream);
  const std::size_t cell = aligned(sizeof(T));
  void* base = nullptr;
  const Scratch answer = ctx.acquire(cell + aligned(need ? need : 1), *lane, &base);
  T host = identity;
  if(answer == Scratch::ok) {
    T* total = static_cast<T*>(base);
    api.reduce(static_cast<char*>(base) + cell, need, in, total, n, fold, identity, lane->stream);
    api.copy(&host, total, sizeof(T), Dir::d2h, lane->stream);
    ctx.release(*lane);
  }
  ctx.give_back(lane);
  if(answer == Scratch::ok) result = host;
  return answer;
}

// The same fold into `out`, a device cell, on a lane lent after the tickets `after...`: nothing reaches the host
// and nothing waits; the ticket returned orders what reads it.
template<class Api, class T, class Op, class F, class... After>
inline Lent<Api> reduce_to(Context<Api>& ctx, T* out, std::size_t n, T identity, Op op, F value, Scratch* answer,
                           const After&... after) noexcept {
  ctx.observed();
  Api& api = ctx.api();
  Lent<Api> t(ctx);
  (t.follow(after.mark()), ...);
  *answer = Scratch::ok;
  if(!n) {
    api.template lanes<1>(1, [=] CR_DEVICE(std::size_t) { *out = identity; }, t.stream(), BLOCK, 1);
    return t;
  }
  const Indexed<T, F> in{value};
  const Binary<T, Op> fold{op};
  std::size_t need = 0;
  api.reduce(nullptr, need, in, out, n, fold, identity, t.stream());
  void* temp = nullptr;
  *answer = ctx.acquire(aligned(need ? need : 1), t.lane(), &temp);
  if(*answer != Scratch::ok) return t;
  api.reduce(temp, need, in, out, n, fold, identity, t.stream());
  ctx.release(t.lane());
  return t;
}

// The fold with its total written to `at`, a device element, on the synchronous lane: nothing crosses to the host,
// and in a held run nothing waits.
template<class Api, class T, class R, class Op, class F>
inline Scratch reduce_into(Context<Api>& ctx, R* at, std::size_t n, T identity, Op op, F value) noexcept {
  Api& api = ctx.api();
  auto* lane = ctx.lend(true);
  Scratch answer = Scratch::ok;
  if(!n) {
    api.template lanes<1>(1, [=] CR_DEVICE(std::size_t) { *at = identity; }, lane->stream, BLOCK, 1);
  } else {
    const Indexed<T, F> in{value};
    const Binary<T, Op> fold{op};
    std::size_t need = 0;
    api.reduce(nullptr, need, in, static_cast<T*>(nullptr), n, fold, identity, lane->stream);
    const std::size_t cell = aligned(sizeof(T));
    void* base = nullptr;
    answer = ctx.acquire(cell + aligned(need ? need : 1), *lane, &base);
    if(answer == Scratch::ok) {
      T* total = static_cast<T*>(base);
      api.reduce(static_cast<char*>(base) + cell, need, in, total, n, fold, identity, lane->stream);
      api.template lanes<1>(1, [=] CR_DEVICE(std::size_t) { *at = *total; }, lane->stream, BLOCK, 1);
      ctx.release(*lane);
    }
  }
  ctx.finish(lane);
  return answer;
}

// Both scans: the inclusive scan of value into arena scratch (so a value(i) that reads out[i] reads it before any
// write), then one pass writing out from it (shifted one place, identity first, when Exclusive), and with `last`
// the total's copy to the host, which the caller's wait completes.
template<bool Exclusive, class Api, class T, class R, class Op, class F>
inline Scratch scanned(Context<Api>& ctx, typename Context<Api>::Lane& lane, T* last, R* out, std::size_t n,
                       T identity, Op op, F value) noexcept {
  Api& api = ctx.api();
  const Indexed<T, F> in{value};
  const Binary<T, Op> fold{op};
  std::size_t need = 0;
  api.inclusive_scan(nullptr, need, in, static_cast<T*>(nullptr), fold, n, lane.stream);
  const std::size_t held = aligned(span<T>(n));
  void* base = nullptr;
  const Scratch answer = ctx.acquire(held + aligned(need ? need : 1), lane, &base);
  if(answer != Scratch::ok) return answer;
  T* h = static_cast<T*>(base);
  api.inclusive_scan(static_cast<char*>(base) + held, need, in, h, fold, n, lane.stream);
  api.template lanes<1>(
      n, [=] CR_DEVICE(std::size_t i) { out[i] = Exclusive ? (i ? h[i - 1] : identity) : h[i]; }, lane.stream, BLOCK,
      1);
  if(last) api.copy(last, h + (n - 1), sizeof(T), Dir::d2h, lane.stream);
  ctx.release(lane);
  return answer;
}
// out[i] = op over value(0 .. i] (Exclusive: over value(0 .. i)), `total` op over all of them, on the host.
template<bool Exclusive, class Api, class T, class R, class Op, class F>
inline Scratch scan(Context<Api>& ctx, T& total, R* out, std::size_t n, T identity, Op op, F value) noexcept {
  if(!n) {
    total = identity;
    return Scratch::ok;
  }
  ctx.observed();
  auto* lane = ctx.lend(true);
  T last = identity;
  const Scratch answer = scanned<Exclusive>(ctx, *lane, &last, out, n, identity, op, value);
  ctx.give_back(lane);
  if(answer == Scratch::ok) total = last;
  return answer;
}
// The same scan with no total for the host: in a held run nothing waits.
template<bool Exclusive, class Api, class T, class R, class Op, class F>
inline Scratch scan_into(Context<Api>& ctx, R* out, std::size_t n, T identity, Op op, F value) noexcept {
  if(!n) return Scratch::ok;
  auto* lane = ctx.lend(true);
  const Scratch answer = scanned<Exclusive>(ctx, *lane, static_cast<T*>(nullptr), out, n, identity, op, value);
  ctx.finish(lane);
  return answer;
}

// Stable compaction: value(i) for each i where pred(i), in order, into the front of out; the rest of out is left
// alone. pred runs once per i, value only where selected. The flags, their exclusive sums and the library's
// storage come from the arena; `*used` is how many were selected (0 when over budget).
template<class Api, class T, class P, class F>
inline Scratch compact(Context<Api>& ctx, std::size_t* used, T* out, std::size_t n, P pred, F value) noexcept {
  *used = 0;
  if(!n) return Scratch::ok;
  ctx.observed();
  Api& api = ctx.api();
  auto* lane = ctx.lend(true);
  std::size_t need = 0;
  api.exclusive_sum(nullptr, need, static_cast<unsigned char*>(nullptr), static_cast<std::size_t*>(nullptr), n,
                    lane->stream);
  const std::size_t flags = aligned(n), offsets = aligned(span<std::size_t>(n));
  void* base = nullptr;
  const Scratch answer = ctx.acquire(flags + offsets + aligned(need ? need : 1), *lane, &base);
  std::size_t last = 0;
  unsigned char tail = 0;
  if(answer == Scratch::ok) {
    unsigned char* k = static_cast<unsigned char*>(base);
    std::size_t* o = reinterpret_cast<std::size_t*>(static_cast<char*>(base) + flags);
    api.template lanes<1>(n, [=] CR_DEVICE(std::size_t i) { k[i] = pred(i) ? 1 : 0; }, lane->stream, BLOCK, 1);
    api.exclusive_sum(static_cast<char*>(base) + flags + offsets, need, k, o, n, lane->stream);
    api.template lanes<1>(
        n, [=] CR_DEVICE(std::size_t i) {
          if(k[i]) out[o[i]] = value(i);
        },
        lane->stream, BLOCK, 1);
    api.copy(&last, o + (n - 1), sizeof(last), Dir::d2h, lane->stream);
    api.copy(&tail, k + (n - 1), sizeof(tail), Dir::d2h, lane->stream);
    ctx.release(*lane);
  }
  ctx.give_back(lane);
  if(answer == Scratch::ok) *used = last + (tail ? 1 : 0);
  return answer;
}

}  // namespace cr::reuse
