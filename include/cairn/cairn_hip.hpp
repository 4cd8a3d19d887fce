// HIP as the machine the execution context (cairn_context.hpp) runs on, for gfx950. Each member is one HIP runtime
// call or one queued kernel; nothing waits for the whole device, streams are made at the default priority, and zeros
// are written by a fill kernel, never hipMemsetAsync, so that an enqueued call stays capturable in a graph. A HIP
// error prints "cairn: hip: <message>" and traps (the reference's check, src/cairn/runtime/cairn_kernels.hpp:55-59,
// prints "cairn: cuda: "); a refusal of the GEMM library prints "cairn: gemm: <status>" and traps.
//
// The members that launch device code (lanes, vector_lanes, staged_lanes, zero, fold, scan) are declared here and
// defined in cairn_hip_kernels.hpp, which hipcc reads through cairn_gpu.hpp: a host-compiled unit that only
// multiplies never needs them. The multiply goes to the gfx950 kernels through the C ABI of libcairn_gemm_gfx950.so.
#pragma once
#include <hip/hip_runtime_api.h>
#include <cstddef>
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
// A release while the process exits may find the runtime already gone: nothing is left to release then.
inline void check_release(hipError_t e) noexcept {
  if(e == hipErrorDeinitialized || e == hipErrorContextIsDestroyed) return;
  check(e);
}

struct Hip {
  using Stream = hipStream_t;
  using Event = hipEvent_t;

  // A C caller's stream handle, as the entries receive it.
  static Stream stream_of(void* handle) noexcept { return static_cast<hipStream_t>(handle); }

  Stream open_stream() noexcept {
    hipStream_t s = nullptr;
    check(hipStreamCreateWithFlags(&s, hipStreamDefault));
    return s;
  }
  void close_stream(Stream s) noexcept { check_release(hipStreamDestroy(s)); }
  Event open_event() noexcept {
    hipEvent_t e = nullptr;
    check(hipEventCreateWithFlags(&e, hipEventDisableTiming));
    return e;
  }
  void close_event(Event e) noexcept { check_release(hipEventDestroy(e)); }
  void mark(Event e, Stream s) noexcept { check(hipEventRecord(e, s)); }
  void after(Stream s, Event e) noexcept { check(hipStreamWaitEvent(s, e, 0)); }
  void drain(Stream s) noexcept { check(hipStreamSynchronize(s)); }
  void drain_event(Event e) noexcept { check_release(hipEventSynchronize(e)); }

  void* take(std::size_t bytes) noexcept {
    void* p = nullptr;
    check(hipMalloc(&p, bytes));
    return p;
  }
  void give(void* p) noexcept { check_release(hipFree(p)); }
  void* take_async(std::size_t bytes, Stream s) noexcept {
    void* p = nullptr;
    check(hipMallocAsync(&p, bytes, s));
    return p;
  }
  void give_async(void* p, Stream s) noexcept { check(hipFreeAsync(p, s)); }
  // An owner's storage: device memory, pinned host memory (allocated pinned: this pool cannot pin memory that already
  // exists), or managed memory.
  void* take_where(reuse::Where w, std::size_t bytes) noexcept {
    void* p = nullptr;
    switch(w) {
      case reuse::Where::device: check(hipMalloc(&p, bytes)); break;
      case reuse::Where::pinned: check(hipHostMalloc(&p, bytes, hipHostMallocDefault)); break;
      case reuse::Where::unified: check(hipMallocManaged(&p, bytes, hipMemAttachGlobal)); break;
    }
    return p;
  }
  void give_where(reuse::Where w, void* p) noexcept { check_release(w == reuse::Where::pinned ? hipHostFree(p) : hipFree(p)); }
  // A copy on the stream; unified addressing tells the runtime which way it goes.
  void copy(void* dst, const void* src, std::size_t bytes, reuse::Dir, Stream s) noexcept {
    check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDefault, s));
  }

  // Device code (cairn_hip_kernels.hpp): bytes of zeros; body(i) for every i below n (one index a lane, W-wide
  // chunks, or a block's tile in LDS); and the fold and inclusive scan of value(i) in a fixed association for n.
  void zero(void* p, std::size_t bytes, Stream s) noexcept;
  template<unsigned U, class F>
  void lanes(std::size_t n, const F& body, Stream s, unsigned block, std::size_t per_lane) noexcept;
  template<unsigned W, unsigned U, class F, class G>
  void vector_lanes(std::size_t n, F scalar, G chunk, Stream s, unsigned block, std::size_t per_lane) noexcept;
  template<std::size_t R, unsigned U, class L, class F, class S>
  void staged_lanes(std::size_t n, L load, F body, S bytes, Stream s, unsigned block, std::size_t per_lane) noexcept;
  template<class T, class F, class Op>
  void fold(std::size_t n, F value, Op op, T identity, T* out, void* work, Stream s) noexcept;
  template<class T, class F, class Op>
  void scan(std::size_t n, F value, Op op, T identity, T* out, void* work, Stream s) noexcept;

  // The fold's first pass gives each of its blocks a run of at least FOLD_RUN indices, at most FOLD_BLOCKS blocks;
  // the partial results (and, for a scan, their running totals) are the scratch the arena provides.
  static constexpr std::size_t FOLD_RUN = 8192;
  static constexpr unsigned FOLD_BLOCKS = 1024;
  static unsigned fold_blocks(std::size_t n) noexcept {
    const std::size_t g = (n + FOLD_RUN - 1) / FOLD_RUN;
    return g < 1 ? 1u : (g > FOLD_BLOCKS ? FOLD_BLOCKS : unsigned(g));
  }
  template<class T> static std::size_t fold_space(std::size_t n) noexcept { return fold_blocks(n) * sizeof(T); }
  template<class T> static std::size_t scan_space(std::size_t n) noexcept { return 2 * fold_blocks(n) * sizeof(T); }

  // The multiply: the reference's c += a b on a stream, and any GEMM the C ABI describes.
  void mma(int type, std::size_t m, std::size_t n, std::size_t k, float* c, const void* a, const void* b,
           Stream s) noexcept {
    check_gemm(cairn_gemm_mma(type, m, n, k, c, a, b, s));
  }
  void gemm(const cairn_gemm_desc& d, Stream s) noexcept { check_gemm(cairn_gemm_run(&d, s)); }
};

using Machine = Hip;

}  // namespace cr::gpu
