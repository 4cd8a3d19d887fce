// HIP as the machine the execution context runs on (the role cairn_gpu.hpp's Cuda machine plays in the reference,
// src/cairn/runtime/cairn_gpu.hpp:47-126): each member is one HIP runtime call, nothing waits for the whole device,
// and nothing makes a stream but make_stream. A HIP error prints "cairn: hip: <message>" and aborts, as the
// reference's check does (cairn_kernels.hpp:55-59). The multiply goes to the gfx950 kernels through the C ABI of
// libcairn_gemm_gfx950.so, whose own failures abort the same way.
//
// With this header included, cr::gpu::here(), use_stream, Held and Enqueued have the meaning emitted code expects
// (src/cairn/runtime/cairn_exec.hpp:25-67).
#pragma once
#include <hip/hip_runtime_api.h>
#include <cstdio>
#include "../cairn_gemm.h"
#include "cairn_context.hpp"
#include "cairn_runtime.hpp"

namespace cr::gpu {

inline void check(hipError_t e) noexcept {
  if(e == hipSuccess) return;
  std::fprintf(stderr, "cairn: hip: %s\n", hipGetErrorString(e));
  trap();
}
inline void check_gemm(int status) noexcept {
  if(status == CAIRN_OK) return;
  std::fprintf(stderr, "cairn: gemm: %s\n", cairn_gemm_status_string(status));
  trap();
}
// A release at process exit may find the HIP runtime already torn down; nothing is left to release then.
inline void released(hipError_t e) noexcept {
  if(e != hipErrorDeinitialized && e != hipErrorContextIsDestroyed) check(e);
}

struct Hip {
  using Stream = hipStream_t;
  using Event = hipEvent_t;
  Stream make_stream() noexcept {
    hipStream_t s = nullptr;
    check(hipStreamCreate(&s));  // default priority, ordered after the null stream's work
    return s;
  }
  void destroy_stream(Stream s) noexcept { released(hipStreamDestroy(s)); }
  Event make_event() noexcept {
    hipEvent_t e = nullptr;
    check(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    return e;
  }
  void destroy_event(Event e) noexcept { released(hipEventDestroy(e)); }
  void record(Event e, Stream s) noexcept { check(hipEventRecord(e, s)); }
  void wait_event(Stream s, Event e) noexcept { check(hipStreamWaitEvent(s, e, 0)); }
  void sync_stream(Stream s) noexcept { check(hipStreamSynchronize(s)); }
  void sync_event(Event e) noexcept { check(hipEventSynchronize(e)); }
  void mma(int type, std::size_t m, std::size_t n, std::size_t k, float* c, const void* a, const void* b,
           Stream s) noexcept {
    check_gemm(cairn_gemm_mma(type, m, n, k, c, a, b, s));
  }
  void gemm(const cairn_gemm_desc& d, Stream s) noexcept { check_gemm(cairn_gemm_run(&d, s)); }
};

using Machine = Hip;
using Context = reuse::Context<Machine>;

// The calling thread's execution context, made by its first device operation and kept for the thread's life.
inline Context& here() noexcept {
  thread_local Context held;
  return held;
}

// A stream the caller owns, for the thread's synchronous device work; null gives the thread its own back.
inline void use_stream(void* stream) noexcept {
  if(stream) here().bind(static_cast<hipStream_t>(stream));
  else here().unbind();
}

// A run of synchronous device work that waits once, at its end.
class Held final {
public:
  Held() noexcept { here().hold(); }
  ~Held() noexcept { here().settle(); }
  Held(const Held&) = delete;
  Held& operator=(const Held&) = delete;
};

// An enqueued entry (cq_NAME): the work queues on the caller's stream and nothing waits for it.
class Enqueued final {
public:
  explicit Enqueued(void* stream) noexcept { here().enqueue(static_cast<hipStream_t>(stream)); }
  ~Enqueued() noexcept { here().leave(); }
  Enqueued(const Enqueued&) = delete;
  Enqueued& operator=(const Enqueued&) = delete;
};

}  // namespace cr::gpu
