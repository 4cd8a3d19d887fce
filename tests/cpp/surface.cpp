// The multiply's C++ surface (include/cairn) on the host, under a machine that records every call instead of running
// HIP. tests/test_cpp_surface.py builds it with g++ and drives it:
//
//   surface context            the execution context's stream, wait and reuse rules; prints one line per check
//   surface trap <case>        one misuse the context refuses; must end in SIGABRT
//   surface narrow <fmt> <in> <out>     cr::fp::narrow<T> of the doubles in <in>, patterns (uint32) to <out>
//   surface quantize <fmt> <in> <out>   cr::fp::quantize<T>(x, scale), (x, scale) float pairs in, patterns out
//   surface decode <fmt> <in> <out>     double(T{bits}) of the uint32 patterns in <in>
//   surface mma <fmt> m n k <a> <b> <c> <out>  cr::tensor::multiply<T> on raw arrays
//
// The context's rules are the semantics CAIRN's generated code relies on (src/cairn/runtime/cairn_reuse.hpp:1-267):
// synchronous work returns once its stream ran it and never waits for the device, a bound stream takes the work after
// what the caller queued, a held run waits once, an enqueued call never waits and makes nothing, tickets keep their
// streams across calls, and the arena passes between users by events.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>
#include "cairn/cairn_tensor.hpp"

namespace {

struct Log {
  int streams = 0, events = 0, destroyed = 0, marks = 0, afters = 0, drains = 0, mmas = 0, gemms = 0;
  int allocs = 0, frees = 0, async_allocs = 0, async_frees = 0, event_drains = 0, lane_runs = 0, library = 0;
  std::vector<int> drained, launched;  // stream names in order
  std::vector<std::size_t> sizes;      // bytes of each allocation, in order
};

// A machine whose streams and events are small integers; every call is counted, and work runs at once on the host.
struct Recorder {
  using Stream = int;
  using Event = int;
  Log* log;
  static Stream stream_of(void* p) noexcept { return int(reinterpret_cast<std::uintptr_t>(p)); }
  Stream open_stream() noexcept { return ++log->streams; }
  void close_stream(Stream) noexcept { ++log->destroyed; }
  Event open_event() noexcept { return ++log->events; }
  void close_event(Event) noexcept {}
  void mark(Event, Stream) noexcept { ++log->marks; }
  void after(Stream, Event) noexcept { ++log->afters; }
  void drain(Stream s) noexcept {
    ++log->drains;
    log->drained.push_back(s);
  }
  void drain_event(Event) noexcept { ++log->event_drains; }
  // Host memory stands for device memory, so the operations run their bodies on it.
  void* take(std::size_t b) noexcept {
    ++log->allocs;
    log->sizes.push_back(b);
    return std::malloc(b);
  }
  void give(void* p) noexcept {
    ++log->frees;
    std::free(p);
  }
  void* take_async(std::size_t b, Stream) noexcept {
    ++log->async_allocs;
    log->sizes.push_back(b);
    return std::malloc(b);
  }
  void give_async(void* p, Stream) noexcept {
    ++log->async_frees;
    std::free(p);
  }
  void copy(void* dst, const void* src, std::size_t b, cr::reuse::Dir, Stream) noexcept { std::memcpy(dst, src, b); }
  template<unsigned U, class F> void lanes(std::size_t n, const F& body, Stream, unsigned, std::size_t) noexcept {
    ++log->lane_runs;
    for(std::size_t i = 0; i < n; ++i) body(i);
  }
  // The fold and scan say they need a few bytes of scratch per value, and use it, so that a scratch part too small or
  // overlapping another would show.
  template<class T> static std::size_t fold_space(std::size_t) noexcept { return 3 * sizeof(T); }
  template<class T> static std::size_t scan_space(std::size_t n) noexcept { return (n + 1) * sizeof(T); }
  template<class T, class F, class Op> void fold(std::size_t n, F value, Op op, T identity, T* out, void* work, Stream) noexcept {
    ++log->library;
    T* w = static_cast<T*>(work);
    w[0] = identity;
    for(std::size_t i = 0; i < n; ++i) w[0] = op(w[0], value(i));
    *out = w[0];
  }
  template<class T, class F, class Op> void scan(std::size_t n, F value, Op op, T identity, T* out, void* work, Stream) noexcept {
    ++log->library;
    T* w = static_cast<T*>(work);
    w[0] = identity;
    for(std::size_t i = 0; i < n; ++i) w[i + 1] = out[i] = w[0] = op(w[0], value(i));
  }
  // The device multiply, run at once on the host arrays: its results are the reference loop's.
  void mma(int type, std::size_t m, std::size_t n, std::size_t k, float* c, const void* a, const void* b,
           Stream s) noexcept {
    ++log->mmas;
    log->launched.push_back(s);
    if(type == CAIRN_TYPE_BF16)
      cr::tensor::reference(m, n, k, c, static_cast<const cr::bf16*>(a), static_cast<const cr::bf16*>(b));
    else cr::trap();
  }
  void gemm(const cairn_gemm_desc&, Stream s) noexcept {
    ++log->gemms;
    log->launched.push_back(s);
  }
};

using Ctx = cr::reuse::Context<Recorder>;
using cr::reuse::Scratch;

int failures = 0;
void expect(bool ok, const char* what) {
  std::printf("%s %s\n", ok ? "ok" : "FAIL", what);
  if(!ok) ++failures;
}

void launch(Ctx& ctx, std::vector<float>& c, const std::vector<cr::bf16>& a, const std::vector<cr::bf16>& b,
            std::size_t m, std::size_t n, std::size_t k) {
  cr::tensor::launch<cr::bf16>(ctx, m, n, k, c.data(), c.size(), a.data(), a.size(), b.data(), b.size());
}

struct Add {
  long long operator()(long long x, long long y) const { return x + y; }
};
struct Index {
  long long operator()(std::size_t i) const { return (long long)i; }
};

int context() {
  const std::size_t m = 3, n = 4, k = 5;
  std::vector<cr::bf16> a(m * k), b(k * n);
  for(std::size_t i = 0; i < a.size(); ++i) a[i] = cr::fp::narrow<cr::bf16>(double(int(i % 7) - 3) / 4);
  for(std::size_t i = 0; i < b.size(); ++i) b[i] = cr::fp::narrow<cr::bf16>(double(int(i % 5) - 2) / 2);
  std::vector<float> want(m * n, 1.0f);
  cr::tensor::multiply<cr::bf16>(m, n, k, want.data(), want.size(), a.data(), a.size(), b.data(), b.size());

  {  // synchronous work: the home stream, made once, drained by each call
    Log log;
    {
      Ctx ctx(Recorder{&log});
      expect(log.streams == 0 && log.events == 0 && log.allocs == 0, "making a context makes nothing");
      std::vector<float> c(m * n, 1.0f);
      launch(ctx, c, a, b, m, n, k);
      expect(c == want, "the device multiply's result is the host multiply's");
      for(int i = 0; i < 9; ++i) launch(ctx, c, a, b, m, n, k);
      expect(log.streams == 1 && ctx.streams_made() == 1, "ten synchronous calls make one stream");
      expect(log.drains == 10 && log.mmas == 10, "each synchronous call waits for its own stream once");
      bool same = true;
      for(int s : log.drained) same &= s == 1;
      expect(same, "the waits are on that stream, never the device");
      expect(ctx.tickets() == 0, "no ticket is out");
      std::vector<float> d(m * n, 1.0f), none;
      std::vector<cr::bf16> empty;
      launch(ctx, d, empty, empty, m, n, 0);
      launch(ctx, none, empty, b, 0, n, k);
      expect(log.mmas == 10 && log.drains == 10 && d == std::vector<float>(m * n, 1.0f),
             "an empty multiply queues nothing and leaves c");
    }
    expect(log.destroyed == 1, "the context releases its stream at its end");
  }
  {  // a bound stream: the work goes there, drained there; no stream is made
    Log log;
    Ctx ctx(Recorder{&log});
    ctx.bind(77);
    std::vector<float> c(m * n, 1.0f);
    launch(ctx, c, a, b, m, n, k);
    launch(ctx, c, a, b, m, n, k);
    expect(log.streams == 0 && log.launched == std::vector<int>({77, 77}) && ctx.bound(), "a bound stream takes synchronous work");
    expect(log.drained == std::vector<int>({77, 77}), "and each call waits on the bound stream");
    ctx.unbind();
    launch(ctx, c, a, b, m, n, k);
    expect(log.streams == 1 && log.launched.back() == 1 && !ctx.bound(), "unbinding gives the thread its own stream back");
  }
  {  // a held run: every call queues on one stream, one wait at the end
    Log log;
    Ctx ctx(Recorder{&log});
    std::vector<float> c(m * n, 1.0f);
    ctx.hold();
    for(int i = 0; i < 4; ++i) launch(ctx, c, a, b, m, n, k);
    expect(log.drains == 0 && log.mmas == 4, "a held run waits for nothing while it runs");
    ctx.observed();
    expect(log.drains == 1, "a host read inside it waits once");
    ctx.observed();
    expect(log.drains == 1, "and not again while nothing new is queued");
    ctx.hold();  // nested: only the outermost end waits
    launch(ctx, c, a, b, m, n, k);
    ctx.settle();
    expect(log.drains == 1, "an inner run's end waits for nothing");
    ctx.settle();
    expect(log.drains == 2 && log.streams == 1, "the outer end waits once more, on the one stream");
    ctx.hold();
    ctx.settle();
    expect(log.drains == 2, "a held run with nothing queued waits for nothing");
  }
  {  // an enqueued call: the caller's stream, never a wait
    Log log;
    Ctx ctx(Recorder{&log});
    std::vector<float> c(m * n, 1.0f);
    ctx.enqueue(55);
    launch(ctx, c, a, b, m, n, k);
    launch(ctx, c, a, b, m, n, k);
    expect(ctx.enqueued(), "inside it the context says so");
    ctx.leave();
    expect(log.drains == 0 && log.streams == 0 && log.events == 0 && log.launched == std::vector<int>({55, 55}),
           "an enqueued call queues on the caller's stream, makes nothing and never waits");
    expect(!ctx.bound() && !ctx.enqueued(), "leaving restores the thread's binding");
  }
  {  // an enqueued call under a bound stream gives that binding back afterwards
    Log log;
    Ctx ctx(Recorder{&log});
    ctx.bind(9);
    ctx.enqueue(10);
    std::vector<float> c(m * n, 1.0f);
    launch(ctx, c, a, b, m, n, k);
    ctx.leave();
    launch(ctx, c, a, b, m, n, k);
    expect(log.launched == std::vector<int>({10, 9}) && log.drained == std::vector<int>({9}),
           "the bound stream is back after an enqueued call");
  }
  {  // gemm is synchronous work like the multiply
    Log log;
    Ctx ctx(Recorder{&log});
    cairn_gemm_desc d{};
    cr::tensor::gemm(ctx, d);
    expect(log.gemms == 1 && log.drains == 1, "gemm is synchronous work, waited for once");
  }
  {  // the arena: a reserve allocated up front and never again within it; each user ordered after the last
    Log log;
    {
      Ctx ctx(cr::reuse::Budget{1024, 4096}, cr::reuse::Allocation::synchronous, Recorder{&log});
      expect(log.allocs == 1 && ctx.capacity() == 1024, "a budget's reserve is allocated when the context is made");
      const int s = ctx.open_sync();
      void* p = nullptr;
      expect(ctx.lease(512, s, &p) == Scratch::ok && p && log.allocs == 1 && log.afters == 0,
             "scratch within the reserve allocates nothing, and its first user follows no one");
      ctx.unlease(s);
      void* q = nullptr;
      expect(ctx.lease(800, s, &q) == Scratch::ok && q == p && log.afters == 1 && log.marks == 1,
             "the next user's stream follows the event the last one's stream marked");
      ctx.unlease(s);
      const int drained = log.event_drains;
      expect(ctx.lease(2000, s, &q) == Scratch::ok && ctx.grown() == 1 && log.frees == 1 && log.allocs == 2 &&
                 log.sizes.back() == 2000 && log.event_drains == drained + 1 && log.afters == 1,
             "growth within the limit waits for the last user, frees, allocates, and owes the new storage no wait");
      ctx.unlease(s);
      void* r = nullptr;
      expect(ctx.lease(5000, s, &r) == Scratch::over_budget && r == nullptr && log.allocs == 2 && ctx.capacity() == 2000,
             "past the limit the answer is over_budget and nothing changes");
      expect(ctx.lease(100, s, &r) == Scratch::ok, "and the arena is still free to lease");
      ctx.unlease(s);
      ctx.close_sync(false);
    }
    expect(log.frees == 2 && log.event_drains >= 2, "the context's end waits for the arena's last user, then frees it");
  }
  {  // stream-ordered growth: the host never waits; the old storage goes on the requesting stream
    Log log;
    Ctx ctx(cr::reuse::Budget{0, cr::reuse::UNBOUNDED}, cr::reuse::Allocation::stream_ordered, Recorder{&log});
    const int s = ctx.open_sync();
    void* p = nullptr;
    ctx.lease(100, s, &p);
    ctx.unlease(s);
    ctx.lease(300, s, &p);
    ctx.unlease(s);
    expect(log.async_allocs == 2 && log.async_frees == 1 && log.allocs == 0 && log.event_drains == 0,
           "stream-ordered growth allocates and frees on the stream and never stops the host");
    ctx.close_sync(false);
  }
  {  // the operations on the arena: their results, and nothing allocated after the first
    Log log;
    Ctx ctx(Recorder{&log});
    long long total = 0;
    const bool r1 = cr::reuse::reduce(ctx, total, 100, 0LL, Add{}, Index{}) == Scratch::ok && total == 4950;
    const int allocs = log.allocs;
    long long again = 0;
    cr::reuse::reduce(ctx, again, 100, 0LL, Add{}, Index{});
    expect(r1 && again == 4950 && log.allocs == allocs, "a reduce's result, and the arena kept for the next one");
    long long none = -1;
    expect(cr::reuse::reduce(ctx, none, 0, 7LL, Add{}, Index{}) == Scratch::ok && none == 7,
           "a reduce over nothing is its identity");
    std::vector<long long> inc(10), exc(10);
    long long t1 = 0, t2 = 0;
    cr::reuse::scan<false>(ctx, t1, inc.data(), 10, 0LL, Add{}, Index{});
    cr::reuse::scan<true>(ctx, t2, exc.data(), 10, 0LL, Add{}, Index{});
    bool sc = t1 == 45 && t2 == 45;
    for(std::size_t i = 0; i < 10; ++i)
      sc &= inc[i] == (long long)(i * (i + 1) / 2) && exc[i] == (long long)(i ? i * (i - 1) / 2 : 0);
    expect(sc, "inclusive and exclusive scans, with the total");
    std::vector<int> out(60, -1);
    std::size_t used = 0;
    int preds = 0;
    struct Even {
      int* calls;
      bool operator()(std::size_t i) const {
        ++*calls;
        return i % 2 == 0;
      }
    };
    struct Ten {
      int operator()(std::size_t i) const { return int(10 * i); }
    };
    cr::reuse::compact(ctx, &used, out.data(), 100, Even{&preds}, Ten{});
    bool cp = used == 50 && preds == 100 && out[50] == -1;
    for(std::size_t j = 0; j < 50; ++j) cp &= out[j] == int(20 * j);
    expect(cp, "a compaction keeps the selected values in order, counts them, runs pred once an index, leaves the rest");
    long long sunk = -1;
    cr::reuse::reduce_into(ctx, &sunk, 5, 0LL, Add{}, Index{});
    expect(sunk == 10, "reduce_into leaves the total where the device reads it");
    int narrow = -1;
    cr::reuse::reduce_into(ctx, &narrow, 5, 0LL, Add{}, Index{});
    expect(narrow == 10, "and lands it as its destination's type");
    long long cell = -1;
    Scratch answer = Scratch::over_budget;
    cr::reuse::Lent<Recorder> t = cr::reuse::reduce_to(ctx, &cell, 20, 0LL, Add{}, Index{}, &answer);
    std::move(t).wait();
    expect(answer == Scratch::ok && cell == 190 && ctx.tickets() == 0, "reduce_to folds on a ticket of its own");
    Ctx tight(cr::reuse::Budget{0, 0}, cr::reuse::Allocation::synchronous, Recorder{&log});
    long long untouched = 7;
    expect(cr::reuse::reduce(tight, untouched, 10, 0LL, Add{}, Index{}) == Scratch::over_budget && untouched == 7 &&
               tight.tickets() == 0,
           "over budget, a reduce queues nothing and leaves its result");
  }
  {  // scans and folds that stay on the device, inside a held run: nothing waits until it ends
    Log log;
    Ctx ctx(Recorder{&log});
    std::vector<long long> pre(6, -1);
    long long sum = -1;
    ctx.hold();
    cr::reuse::scan_into<true>(ctx, pre.data(), 6, 0LL, Add{}, Index{});
    cr::reuse::reduce_into(ctx, &sum, 6, 0LL, Add{}, Index{});
    expect(log.drains == 0, "device-resident scans and folds in a held run wait for nothing");
    ctx.settle();
    expect(log.drains == 1 && sum == 15 && pre[5] == 10 && pre[0] == 0, "the run's end waits once");
  }
  {  // tickets: a stream each for queued work, ordered after another by its marker, handed back by its one wait
    Log log;
    Ctx ctx(Recorder{&log});
    cr::reuse::Lent<Recorder> first(ctx);
    cr::reuse::Lent<Recorder> second(ctx);
    second.follow(first.mark());
    expect(ctx.tickets() == 2 && first.stream() != second.stream() && log.afters == 1, "two tickets, two streams, one ordered");
    std::move(second).wait();
    std::move(first).wait();
    expect(ctx.tickets() == 0 && ctx.streams_made() == 2, "each wait hands its stream back");
    cr::reuse::Lent<Recorder> third(ctx);
    expect(ctx.streams_made() == 2, "and the next ticket reuses one");
    std::move(third).wait();
  }
  {  // a ticket taken while a run is held, or a stream bound, starts after what was queued there
    Log log;
    Ctx ctx(Recorder{&log});
    std::vector<float> c(m * n, 1.0f);
    ctx.hold();
    launch(ctx, c, a, b, m, n, k);
    cr::reuse::Lent<Recorder> other(ctx);
    expect(log.marks == 1 && log.afters == 1 && other.stream() == 2, "a ticket follows the held run's work");
    std::move(other).wait();
    ctx.settle();
    Log bound_log;
    Ctx bound(Recorder{&bound_log});
    bound.bind(31);
    cr::reuse::Lent<Recorder> after_bound(bound);
    expect(bound_log.marks == 1 && bound_log.afters == 1, "a ticket follows the bound stream's work");
    std::move(after_bound).wait();
  }
  std::printf("%d failures\n", failures);
  return failures ? 1 : 0;
}

int trap_case(const std::string& which) {
  Log log;
  Ctx* ctx = new Ctx(Recorder{&log});  // leaked on purpose: a trap ends the process first
  std::vector<float> c(6);
  std::vector<cr::bf16> a(6), b(9);
  if(which == "shape") cr::tensor::launch<cr::bf16>(*ctx, 2, 3, 3, c.data(), c.size(), a.data(), a.size(), b.data(), 8);
  else if(which == "nested") {
    ctx->open_sync();
    ctx->open_sync();  // synchronous work does not nest
  } else if(which == "settle") ctx->settle();  // no run held
  else if(which == "observe") {
    ctx->enqueue(3);
    ctx->observed();  // a wait inside an enqueued call
  } else if(which == "leaked") {
    ctx->lend();
    delete ctx;  // a ticket never given back
  } else if(which == "lease") {  // the arena leased twice
    const int s = ctx->open_sync();
    void* p = nullptr;
    ctx->lease(16, s, &p);
    ctx->lease(16, s, &p);
  } else if(which == "unleased") {  // handed back with no lease
    ctx->unlease(ctx->open_sync());
  } else if(which == "ticket") {  // a ticket dropped unawaited
    cr::reuse::Lent<Recorder> t(*ctx);
  } else if(which == "rebind") {  // a binding changed under a held run with work pending
    std::vector<float> d(6, 0.0f);
    std::vector<cr::bf16> x(6), y(9);
    ctx->hold();
    cr::tensor::launch<cr::bf16>(*ctx, 2, 3, 3, d.data(), d.size(), x.data(), x.size(), y.data(), y.size());
    ctx->bind(4);
  } else if(which == "overflow") (void)cr::mul<std::size_t>(std::size_t(1) << 40, std::size_t(1) << 40);
  else if(which == "e4m3") (void)cr::fp::narrow<cr::f8e4m3>(465.0);
  else if(which == "scale") (void)cr::fp::quantize<cr::bf16>(1.0f, 0.0f);
  std::printf("returned\n");
  return 0;
}

template<class F> std::vector<F> read(const char* path) {
  std::FILE* f = std::fopen(path, "rb");
  if(!f) std::exit(3);
  std::vector<F> v;
  F x;
  while(std::fread(&x, sizeof x, 1, f) == 1) v.push_back(x);
  std::fclose(f);
  return v;
}
template<class F> void write(const char* path, const std::vector<F>& v) {
  std::FILE* f = std::fopen(path, "wb");
  if(!f) std::exit(3);
  if(!v.empty() && std::fwrite(v.data(), sizeof(F), v.size(), f) != v.size()) std::exit(3);
  std::fclose(f);
}

template<class T> int storage(const std::string& op, char** argv) {
  if(op == "narrow") {
    std::vector<std::uint32_t> out;
    for(double x : read<double>(argv[0])) out.push_back(cr::fp::narrow<T>(x).bits);
    write(argv[1], out);
  } else if(op == "quantize") {
    const auto xs = read<float>(argv[0]);
    std::vector<std::uint32_t> out;
    for(std::size_t i = 0; i + 1 < xs.size(); i += 2) out.push_back(cr::fp::quantize<T>(xs[i], xs[i + 1]).bits);
    write(argv[1], out);
  } else if(op == "decode") {
    std::vector<double> out;
    for(std::uint32_t p : read<std::uint32_t>(argv[0])) out.push_back(double(T{typename T::Bits(p)}));
    write(argv[1], out);
  } else if(op == "mma") {
    const std::size_t m = std::strtoull(argv[0], nullptr, 10), n = std::strtoull(argv[1], nullptr, 10),
                      k = std::strtoull(argv[2], nullptr, 10);
    const auto a = read<T>(argv[3]);
    const auto b = read<T>(argv[4]);
    auto c = read<float>(argv[5]);
    cr::tensor::multiply<T>(m, n, k, c.data(), c.size(), a.data(), a.size(), b.data(), b.size());
    write(argv[6], c);
  } else return 2;
  return 0;
}

}  // namespace

int main(int argc, char** argv) {
  if(argc < 2) return 2;
  const std::string op = argv[1];
  if(op == "context") return context();
  if(op == "trap" && argc == 3) return trap_case(argv[2]);
  if(argc < 5) return 2;
  const std::string fmt = argv[2];
  if(fmt == "f16") return storage<cr::f16>(op, argv + 3);
  if(fmt == "bf16") return storage<cr::bf16>(op, argv + 3);
  if(fmt == "f8e4m3") return storage<cr::f8e4m3>(op, argv + 3);
  if(fmt == "f8e5m2") return storage<cr::f8e5m2>(op, argv + 3);
  return 2;
}
