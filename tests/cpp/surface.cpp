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
  std::vector<int> synced, launched;  // stream ids in order
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
  void sync_event(Event) noexcept {}
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
