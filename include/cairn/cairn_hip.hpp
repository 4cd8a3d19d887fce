// HIP as the machine the execution context runs on (the role cairn_gpu.hpp's Cuda machine plays in the reference,
// src/cairn/runtime/cairn_gpu.hpp:47-126): each member is one HIP runtime call, nothing waits for the whole device,
// and nothing makes a stream but make_stream. A HIP error prints "cairn: hip: <message>" and aborts, as the
// reference's check does (cairn_kernels.hpp:55-59). The multiply goes to the gfx950 kernels through the C ABI of
// libcairn_gemm_gfx950.so, whose own failures abort the same way.
//
// The members that launch device code (lanes, vector_lanes, staged_lanes) and those of the device library (reduce,
// inclusive_scan, exclusive_sum, on hipCUB) are declared here and defined in cairn_hip_exec.hpp, which a program
// with device regions includes (through cairn_gpu.hpp): a translation unit that only multiplies never reads them.
//
// With this header included, cr::gpu::here(), use_stream, Held and Enqueued have the meaning emitted code expects
// (src/cairn/runtime/cairn_exec.hpp:25-67).
#pragma once
#include <hip/hip_runtime_api.h>
#include <cstdint>
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
  // A stream's name for the life of the process (its handle), its id among the streams alive now, and whether it
  // is capturing into a graph (with the capture sequence's id).
  unsigned long long handle(Stream s) noexcept { return reinterpret_cast<std::uintptr_t>(s); }
  unsigned long long stream_id(Stream s) noexcept {
    unsigned long long id = 0;
    check(hipStreamGetId(s, &id));
    return id;
  }
  bool capturing(Stream s, unsigned long long* id) noexcept {
    hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
    check(hipStreamGetCaptureInfo(s, &status, id));
    return status != hipStreamCaptureStatusNone;
  }
  void sync_stream(Stream s) noexcept { check(hipStreamSynchronize(s)); }
  void sync_event(Event e) noexcept { released(hipEventSynchronize(e)); }
  // Device memory at once, or ordered on a stream (hipMallocAsync's pool); storage by where it lives: device, pinned
  // host memory (hipHostMalloc: this pool cannot register memory that already exists), or unified.
  void* alloc(std::size_t b) noexcept {
    void* p = nullptr;
    check(hipMalloc(&p, b));
    return p;
  }
  void free(void* p) noexcept { released(hipFree(p)); }
  void* alloc_async(std::size_t b, Stream s) noexcept {
    void* p = nullptr;
    check(hipMallocAsync(&p, b, s));
    return p;
  }
  void free_async(void* p, Stream s) noexcept { check(hipFreeAsync(p, s)); }
  void* allocate(reuse::Where w, std::size_t b) noexcept {
    void* p = nullptr;
    if(w == reuse::Where::device) check(hipMalloc(&p, b));
    else if(w == reuse::Where::pinned) check(hipHostMalloc(&p, b, hipHostMallocDefault));
    else check(hipMallocManaged(&p, b, hipMemAttachGlobal));
    return p;
  }
  void release(reuse::Where w, void* p) noexcept { check(w == reuse::Where::pinned ? hipHostFree(p) : hipFree(p)); }
  // b bytes of zeros at p, queued on the stream by a fill kernel (defined in cairn_hip_exec.hpp), never by
  // hipMemsetAsync, whose graph nodes a captured call must not hold; and a copy queued on the stream.
  void zero(void* p, std::size_t b, Stream s) noexcept;
  void copy(void* dst, const void* src, std::size_t b, reuse::Dir d, Stream s) noexcept {
    check(hipMemcpyAsync(dst, src, b, kind(d), s));
  }
  static hipMemcpyKind kind(reuse::Dir d) noexcept {
    switch(d) {
      case reuse::Dir::h2d: return hipMemcpyHostToDevice;
      case reuse::Dir::d2h: return hipMemcpyDeviceToHost;
      case reuse::Dir::d2d: return hipMemcpyDeviceToDevice;
      case reuse::Dir::h2h: return hipMemcpyHostToHost;
    }
    trap();
  }
  // Defined in cairn_hip_exec.hpp: body(i) for every i below n; W-wide chunks with the tail one at a time; a block's
  // tile in LDS between two barriers; and the device library's fold, scan and exclusive sum (each asked first, with
  // null storage, for the bytes of temporary storage it needs).
  template<unsigned U, class F>
  void lanes(std::size_t n, const F& body, Stream s, unsigned block, std::size_t per_lane) noexcept;
  template<unsigned W, unsigned U, class F, class G>
  void vector_lanes(std::size_t n, F scalar, G chunk, Stream s, unsigned block, std::size_t per_lane) noexcept;
  template<std::size_t R, unsigned U, class L, class F, class S>
  void staged_lanes(std::size_t n, L load, F body, S bytes, Stream s, unsigned block, std::size_t per_lane) noexcept;
  template<class In, class Out, class Fold, class T>
  void reduce(void* temp, std::size_t& bytes, In in, Out out, std::size_t n, Fold fold, T identity, Stream s) noexcept;
  template<class In, class Out, class Fold>
  void inclusive_scan(void* temp, std::size_t& bytes, In in, Out out, Fold fold, std::size_t n, Stream s) noexcept;
  template<class In, class Out>
  void exclusive_sum(void* temp, std::size_t& bytes, In in, Out out, std::size_t n, Stream s) noexcept;
  void mma(int type, std::size_t m, std::size_t n, std::size_t k, float* c, const void* a, const void* b,
           Stream s) noexcept {
    check_gemm(cairn_gemm_mma(type, m, n, k, c, a, b, s));
  }
  void gemm(const cairn_gemm_desc& d, Stream s) noexcept { check_gemm(cairn_gemm_run(&d, s)); }
};

using Machine = Hip;
using Context = reuse::Context<Machine>;
using Lent = reuse::Lent<Machine>;
using reuse::Allocation;
using reuse::Budget;
using reuse::Dir;
using reuse::Scratch;
using reuse::Where;

// The calling thread's execution context, made by its first device operation and kept for the thread's life. Its
// budget lets the arena grow to the largest request met so far, and keeps it, so a pipeline run again allocates no
// scratch.
inline Context& here() noexcept {
  thread_local Context held(Budget{0, reuse::UNBOUNDED});
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
