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
// The context rules follow src/cairn/runtime/cairn_reuse.hpp:57-200 and the reference's own tests of them
// (tests/runtime/reuse_runtime.cpp): synchronous work returns once its stream ran it and never waits for the device,
// a bound stream takes the work after what the caller queued, a held run waits once, an enqueued call never waits,
// lanes are kept across calls.
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>
#include "cairn/cairn_tensor.hpp"

namespace {

struct Log {
  int streams = 0, events = 0, destroyed = 0, records = 0, waits = 0, syncs = 0, mmas = 0, gemms = 0;
  int allocs = 0, frees = 0, async_allocs = 0, async_frees = 0, event_syncs = 0, lane_runs = 0, library = 0;
  std::vector<int> synced, launched;  // stream ids in order
  std::vector<std::size_t> sizes;     // bytes of each allocation, in order
};

// A machine whose streams are small integers; every call is counted.
struct Recorder {
  using Stream = int;
  using Event = int;
  Log* log;
  Stream make_stream() noexcept { return ++log->streams; }
  void destroy_stream(Stream) noexcept { ++log->destroyed; }
  Event make_event() noexcept { return ++log->events; }
  void destroy_event(Event) noexcept {}
  void record(Event, Stream) noexcept { ++log->records; }
  void wait_event(Stream, Event) noexcept { ++log->waits; }
  void sync_stream(Stream s) noexcept {
    ++log->syncs;
    log->synced.push_back(s);
  }
  void sync_event(Event) noexcept { ++log->event_syncs; }
  // Memory: host memory stands for device memory, so the operations run their bodies on it.
  void* alloc(std::size_t b) noexcept {
    ++log->allocs;
    log->sizes.push_back(b);
    return std::malloc(b);
  }
  void free(void* p) noexcept {
    ++log->frees;
    std::free(p);
  }
  void* alloc_async(std::size_t b, Stream) noexcept {
    ++log->async_allocs;
    log->sizes.push_back(b);
    return std::malloc(b);
  }
  void free_async(void* p, Stream) noexcept {
    ++log->async_frees;
    std::free(p);
  }
  void copy(void* dst, const void* src, std::size_t b, cr::reuse::Dir, Stream) noexcept { std::memcpy(dst, src, b); }
  // The lane and library primitives, run at once on the host: body(i) for every i; a fold, an inclusive scan and an
  // exclusive sum that, asked with null storage, say they need a few bytes of it.
  template<unsigned U, class F> void lanes(std::size_t n, const F& body, Stream, unsigned, std::size_t) noexcept {
    ++log->lane_runs;
    for(std::size_t i = 0; i < n; ++i) body(i);
  }
  template<class In, class Out, class Fold, class T>
  void reduce(void* temp, std::size_t& bytes, In in, Out out, std::size_t n, Fold fold, T identity, Stream) noexcept {
    if(!temp) {
      bytes = 96;
      return;
    }
    ++log->library;
    T acc = identity;
    for(std::size_t i = 0; i < n; ++i) acc = fold(acc, in[i]);
    *out = acc;
  }
  template<class In, class Out, class Fold>
  void inclusive_scan(void* temp, std::size_t& bytes, In in, Out out, Fold fold, std::size_t n, Stream) noexcept {
    if(!temp) {
      bytes = 40;
      return;
    }
    ++log->library;
    auto acc = in[0];
    out[0] = acc;
    for(std::size_t i = 1; i < n; ++i) out[i] = acc = fold(acc, in[i]);
  }
  template<class In, class Out>
  void exclusive_sum(void* temp, std::size_t& bytes, In in, Out out, std::size_t n, Stream) noexcept {
    if(!temp) {
      bytes = 24;
      return;
    }
    ++log->library;
    std::size_t acc = 0;
    for(std::size_t i = 0; i < n; ++i) {
      out[i] = acc;
      acc += in[i];
    }
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

int failures = 0;
void expect(bool ok, const char* what) {
  std::printf("%s %s\n", ok ? "ok" : "FAIL", what);
  if(!ok) ++failures;
}

void launch(Ctx& ctx, std::vector<float>& c, const std::vector<cr::bf16>& a, const std::vector<cr::bf16>& b,
            std::size_t m, std::size_t n, std::size_t k) {
  cr::tensor::launch<cr::bf16>(ctx, m, n, k, c.data(), c.size(), a.data(), a.size(), b.data(), b.size());
}

int context() {
  const std::size_t m = 3, n = 4, k = 5;
  std::vector<cr::bf16> a(m * k), b(k * n);
  for(std::size_t i = 0; i < a.size(); ++i) a[i] = cr::fp::narrow<cr::bf16>(double(int(i % 7) - 3) / 4);
  for(std::size_t i = 0; i < b.size(); ++i) b[i] = cr::fp::narrow<cr::bf16>(double(int(i % 5) - 2) / 2);
  std::vector<float> want(m * n, 1.0f);
  cr::tensor::multiply<cr::bf16>(m, n, k, want.data(), want.size(), a.data(), a.size(), b.data(), b.size());

  {  // synchronous work: one lane, made once, waited on by its own stream each call
    Log log;
    {
      Ctx ctx(Recorder{&log});
      std::vector<float> c(m * n, 1.0f);
      launch(ctx, c, a, b, m, n, k);
      expect(c == want, "the device multiply's result is the host multiply's");
      for(int i = 0; i < 9; ++i) launch(ctx, c, a, b, m, n, k);
      expect(log.streams == 1 && ctx.streams_made() == 1, "ten synchronous calls make one stream");
      expect(log.syncs == 10 && log.mmas == 10, "each synchronous call waits for its own stream once");
      bool same = true;
      for(int s : log.synced) same &= s == 1;
      expect(same, "the waits are on that stream, never the device");
      expect(ctx.lent() == 0, "no lane stays lent");
      std::vector<float> d(m * n, 1.0f), none;
      std::vector<cr::bf16> empty;
      launch(ctx, d, empty, empty, m, n, 0);
      launch(ctx, none, empty, b, 0, n, k);
      expect(log.mmas == 10 && log.syncs == 10 && d == std::vector<float>(m * n, 1.0f),
             "an empty multiply queues nothing and leaves c");
    }
    expect(log.destroyed == 1, "the context releases its lane at its end");
  }
  {  // a bound stream: the work goes there, waited on there; no stream is made
    Log log;
    Ctx ctx(Recorder{&log});
    ctx.bind(77);
    std::vector<float> c(m * n, 1.0f);
    launch(ctx, c, a, b, m, n, k);
    launch(ctx, c, a, b, m, n, k);
    expect(log.streams == 0 && log.launched == std::vector<int>({77, 77}), "a bound stream takes synchronous work");
    expect(log.synced == std::vector<int>({77, 77}), "and each call waits on the bound stream");
    ctx.unbind();
    launch(ctx, c, a, b, m, n, k);
    expect(log.streams == 1 && log.launched.back() == 1, "unbinding gives the thread its own lane back");
  }
  {  // a held run: every call queues on one lane, one wait at the end
    Log log;
    Ctx ctx(Recorder{&log});
    std::vector<float> c(m * n, 1.0f);
    ctx.hold();
    for(int i = 0; i < 4; ++i) launch(ctx, c, a, b, m, n, k);
    expect(log.syncs == 0 && log.mmas == 4, "a held run waits for nothing while it runs");
    ctx.observed();
    expect(log.syncs == 1, "a host read inside it waits once");
    launch(ctx, c, a, b, m, n, k);
    ctx.settle();
    expect(log.syncs == 2 && log.streams == 1, "its end waits once more, on the one lane");
  }
  {  // an enqueued call: the caller's stream, never a wait
    Log log;
    Ctx ctx(Recorder{&log});
    std::vector<float> c(m * n, 1.0f);
    ctx.enqueue(55);
    launch(ctx, c, a, b, m, n, k);
    launch(ctx, c, a, b, m, n, k);
    ctx.leave();
    expect(log.syncs == 0 && log.streams == 0 && log.launched == std::vector<int>({55, 55}),
           "an enqueued call queues on the caller's stream and never waits");
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
    expect(log.launched == std::vector<int>({10, 9}) && log.synced == std::vector<int>({9}),
           "the bound stream is back after an enqueued call");
  }
  {  // gemm goes through the same lane
    Log log;
    Ctx ctx(Recorder{&log});
    cairn_gemm_desc d{};
    cr::tensor::gemm(ctx, d);
    expect(log.gemms == 1 && log.syncs == 1, "gemm is synchronous work on the lane");
  }
  {  // the arena: a reserve allocated up front and never again within it; each user waits for the last one
    Log log;
    {
      Ctx ctx(cr::reuse::Budget{1024, 4096}, cr::reuse::Allocation::synchronous, Recorder{&log});
      expect(log.allocs == 1 && ctx.capacity() == 1024, "a budget's reserve is allocated when the context is made");
      auto* lane = ctx.lend(true);
      void* p = nullptr;
      expect(ctx.acquire(512, *lane, &p) == cr::reuse::Scratch::ok && p && log.allocs == 1 && log.waits == 0,
             "scratch within the reserve allocates nothing, and the first user waits for no one");
      ctx.release(*lane);
      void* q = nullptr;
      expect(ctx.acquire(800, *lane, &q) == cr::reuse::Scratch::ok && q == p && log.waits == 1,
             "the next user's stream waits on the event the last one's release recorded");
      ctx.release(*lane);
      const int syncs = log.event_syncs;
      expect(ctx.acquire(2000, *lane, &q) == cr::reuse::Scratch::ok && ctx.grown() == 1 && log.frees == 1 &&
                 log.allocs == 2 && log.sizes.back() == 2000 && log.event_syncs == syncs + 1 && log.waits == 1,
             "growth within the limit waits for the last user, frees, allocates, and owes the new storage no wait");
      ctx.release(*lane);
      void* r = nullptr;
      expect(ctx.acquire(5000, *lane, &r) == cr::reuse::Scratch::over_budget && r == nullptr && log.allocs == 2 &&
                 ctx.capacity() == 2000,
             "past the limit the answer is over_budget and nothing changes");
      expect(ctx.acquire(100, *lane, &r) == cr::reuse::Scratch::ok, "and the arena is still free to lease");
      ctx.release(*lane);
      ctx.give_back(lane);
    }
    expect(log.frees == 2 && log.event_syncs >= 2, "the context's end waits for the arena's last user, then frees it");
  }
  {  // stream-ordered growth: the host never waits, the old storage goes on the lane's stream
    Log log;
    Ctx ctx(cr::reuse::Budget{0, cr::reuse::UNBOUNDED}, cr::reuse::Allocation::stream_ordered, Recorder{&log});
    auto* lane = ctx.lend(true);
    void* p = nullptr;
    ctx.acquire(100, *lane, &p);
    ctx.release(*lane);
    ctx.acquire(300, *lane, &p);
    ctx.release(*lane);
    expect(log.async_allocs == 2 && log.async_frees == 1 && log.allocs == 0 && log.event_syncs == 0,
           "stream-ordered growth allocates and frees on the stream and never stops the host");
    ctx.give_back(lane);
  }
  {  // the operations on the arena: their results, and nothing allocated after the first
    Log log;
    Ctx ctx(Recorder{&log});
    long long total = 0;
    auto value = [](std::size_t i) { return (long long)(i); };
    auto add = [](long long x, long long y) { return x + y; };
    const bool r1 = cr::reuse::reduce(ctx, total, 100, 0LL, add, value) == cr::reuse::Scratch::ok && total == 4950;
    const int allocs = log.allocs;
    long long again = 0;
    cr::reuse::reduce(ctx, again, 100, 0LL, add, value);
    expect(r1 && again == 4950 && log.allocs == allocs, "a reduce's result, and the arena kept for the next one");
    std::vector<long long> inc(10), exc(10);
    long long t1 = 0, t2 = 0;
    cr::reuse::scan<false>(ctx, t1, inc.data(), 10, 0LL, add, value);
    cr::reuse::scan<true>(ctx, t2, exc.data(), 10, 0LL, add, value);
    bool sc = t1 == 45 && t2 == 45;
    for(std::size_t i = 0; i < 10; ++i)
      sc &= inc[i] == (long long)(i * (i + 1) / 2) && exc[i] == (long long)(i ? i * (i - 1) / 2 : 0);
    expect(sc, "inclusive and exclusive scans, with the total");
    std::vector<int> out(50, -1);
    std::size_t used = 0;
    cr::reuse::compact(ctx, &used, out.data(), 100, [](std::size_t i) { return i % 2 == 0; },
                       [](std::size_t i) { return int(10 * i); });
    bool cp = used == 50;
    for(std::size_t j = 0; j < 50; ++j) cp &= out[j] == int(20 * j);
    expect(cp, "a compaction keeps the selected values in order and counts them");
    long long sunk = -1;
    cr::reuse::reduce_into(ctx, &sunk, 5, 0LL, add, value);
    expect(sunk == 10, "reduce_into leaves the total where the device reads it");
    Ctx tight(cr::reuse::Budget{0, 0}, cr::reuse::Allocation::synchronous, Recorder{&log});
    long long untouched = 7;
    expect(cr::reuse::reduce(tight, untouched, 10, 0LL, add, value) == cr::reuse::Scratch::over_budget &&
               untouched == 7 && tight.lent() == 0,
           "over budget, a reduce queues nothing, leaves its result, and gives its lane back");
  }
  {  // tickets: a lent lane for queued work, ordered after another, handed back by its one wait
    Log log;
    Ctx ctx(Recorder{&log});
    cr::reuse::Lent<Recorder> first(ctx);
    cr::reuse::Lent<Recorder> second(ctx);
    second.follow(first.mark());
    expect(ctx.lent() == 2 && first.stream() != second.stream() && log.waits == 1, "two tickets, two lanes, one ordered");
    std::move(second).wait();
    std::move(first).wait();
    expect(ctx.lent() == 0 && ctx.streams_made() == 2, "each wait hands its lane back");
  }
  {  // a second lane while a run is held starts after the held work
    Log log;
    Ctx ctx(Recorder{&log});
    std::vector<float> c(m * n, 1.0f);
    ctx.hold();
    launch(ctx, c, a, b, m, n, k);
    auto* other = ctx.lend();
    expect(log.records == 1 && log.waits == 1 && other->stream == 2, "another lane waits for the held run's work");
    ctx.give_back(other);
    ctx.settle();
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
    ctx->bind(5);
    auto* lane = ctx->lend(true);
    (void)lane;
    ctx->lend(true);  // a second synchronous lane on a bound stream while the first is out
  } else if(which == "settle") ctx->settle();  // no run held
  else if(which == "observe") {
    ctx->enqueue(3);
    ctx->observed();  // a wait inside an enqueued call
  } else if(which == "leaked") {
    ctx->lend();
    delete ctx;  // a lane never given back
  } else if(which == "lease") {  // the arena leased twice
    auto* lane = ctx->lend(true);
    void* p = nullptr;
    ctx->acquire(16, *lane, &p);
    ctx->acquire(16, *lane, &p);
  } else if(which == "unleased") {  // released with no lease
    auto* lane = ctx->lend(true);
    ctx->release(*lane);
  } else if(which == "ticket") {  // a ticket dropped unawaited
    cr::reuse::Lent<Recorder> t(*ctx);
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
