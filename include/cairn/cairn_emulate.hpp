// The emulated machine: device work of a CAIRN program run on the host, for a build without a GPU (`cairn build
// --emulate`, which defines CAIRN_EMULATE and builds with the host compiler: src/cairn/projects/toolchain.py:175-180).
// cairn_gpu.hpp chooses it in place of HIP, and the same context, operations and multiply entries run over it. It is
// a correctness tool, not a way to time device code.
//
// Everything runs to completion when it is queued, in program order, on the calling thread: streams and events are
// names, waits have nothing left to wait for. Device, pinned and unified memory are host memory of the bytes asked
// for (on 256 bytes), so the host's sanitizers see a device array's bounds. Regions run their indices in order; a
// fold and a scan go through the indices in increasing order. The tensor-core multiply is the host's reference loop,
// every product then every sum in increasing k (src/cairn/runtime/cairn_emulate.hpp:151-156), and a GEMM the C ABI
// describes is the same loop in its layout followed by the epilogue's steps in their stated order.
#pragma once
#if !defined(CAIRN_EMULATE) || defined(__HIPCC__)
#error "cairn_emulate.hpp runs device work on the host: build with the host compiler and -DCAIRN_EMULATE"
#endif
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <vector>
#include "../cairn_gemm.h"
#include "cairn_context.hpp"
#include "cairn_float.hpp"
#include "cairn_runtime.hpp"
#include "cairn_tensor.hpp"

namespace cr::gpu {

inline void check_gemm(int status) noexcept {
  if(status != CAIRN_OK) trap();
}

struct Emulated {
  using Stream = std::uintptr_t;
  using Event = std::uintptr_t;
  std::uintptr_t names = 0;

  static Stream stream_of(void* handle) noexcept { return reinterpret_cast<std::uintptr_t>(handle); }
  Stream open_stream() noexcept { return ++names; }
  void close_stream(Stream) noexcept {}
  Event open_event() noexcept { return ++names; }
  void close_event(Event) noexcept {}
  void mark(Event, Stream) noexcept {}
  void after(Stream, Event) noexcept {}
  void drain(Stream) noexcept {}
  void drain_event(Event) noexcept {}

  void* take(std::size_t bytes) noexcept {
    void* p = std::aligned_alloc(256, (bytes + 255) / 256 * 256);
    if(!p) trap();
    return p;
  }
  void give(void* p) noexcept { std::free(p); }
  void* take_async(std::size_t bytes, Stream) noexcept { return take(bytes); }
  void give_async(void* p, Stream) noexcept { give(p); }
  void* take_where(reuse::Where, std::size_t bytes) noexcept { return take(bytes); }
  void give_where(reuse::Where, void* p) noexcept { give(p); }
  void copy(void* dst, const void* src, std::size_t bytes, reuse::Dir, Stream) noexcept { std::memmove(dst, src, bytes); }
  void zero(void* p, std::size_t bytes, Stream) noexcept { std::memset(p, 0, bytes); }

  template<unsigned U, class F> void lanes(std::size_t n, const F& body, Stream, unsigned, std::size_t) noexcept {
    for(std::size_t i = 0; i < n; ++i) body(i);
  }
  template<unsigned W, unsigned U, class F, class G>
  void vector_lanes(std::size_t n, F scalar, G chunk, Stream, unsigned, std::size_t) noexcept {
    for(std::size_t i = 0; i < n; i += W) {
      if(i + W <= n) chunk(i);
      else
        for(std::size_t j = i; j < n; ++j) scalar(j);
    }
  }
  // Each tile loaded whole (every thread's part) before any thread of it runs, as the device's barrier orders it.
  template<std::size_t R, unsigned U, class L, class F, class S>
  void staged_lanes(std::size_t n, L load, F body, S bytes, Stream, unsigned block, std::size_t) noexcept {
    const std::size_t width = block ? block : reuse::BLOCK, halo = width + 2 * R;
    std::vector<unsigned char> tile(bytes(halo) + 16);
    for(std::size_t base = 0; base < n; base += width) {
      for(std::size_t t = 0; t < width; ++t) load(base, halo, t, width, tile.data());
      for(std::size_t t = 0; t < width && base + t < n; ++t) body(base + t, base, halo, tile.data());
    }
  }
  template<class T> static std::size_t fold_space(std::size_t) noexcept { return 0; }
  template<class T> static std::size_t scan_space(std::size_t) noexcept { return 0; }
  template<class T, class F, class Op> void fold(std::size_t n, F value, Op op, T identity, T* out, void*, Stream) noexcept {
    T acc = identity;
    for(std::size_t i = 0; i < n; ++i) acc = op(acc, value(i));
    *out = acc;
  }
  template<class T, class F, class Op> void scan(std::size_t n, F value, Op op, T identity, T* out, void*, Stream) noexcept {
    T acc = identity;
    for(std::size_t i = 0; i < n; ++i) out[i] = acc = op(acc, value(i));
  }

  void mma(int type, std::size_t m, std::size_t n, std::size_t k, float* c, const void* a, const void* b,
           Stream) noexcept {
    switch(type) {
      case CAIRN_TYPE_F16: return multiplied(m, n, k, c, static_cast<const cr::f16*>(a), static_cast<const cr::f16*>(b));
      case CAIRN_TYPE_BF16: return multiplied(m, n, k, c, static_cast<const cr::bf16*>(a), static_cast<const cr::bf16*>(b));
      case CAIRN_TYPE_F8E4M3:
        return multiplied(m, n, k, c, static_cast<const cr::f8e4m3*>(a), static_cast<const cr::f8e4m3*>(b));
      case CAIRN_TYPE_F8E5M2:
        return multiplied(m, n, k, c, static_cast<const cr::f8e5m2*>(a), static_cast<const cr::f8e5m2*>(b));
      default: trap();
    }
  }
  template<class A> static void multiplied(std::size_t m, std::size_t n, std::size_t k, float* c, const A* a,
                                           const A* b) noexcept {
    if(m && n && k) tensor::reference(m, n, k, c, a, b);
  }

  // A descriptor's GEMM on the host: for each output its products in increasing p (f32, or exact int32 for int8),
  // then the epilogue's steps, each an f32 rounding, in the order cairn_gemm.h states, and the output's rounding.
  void gemm(const cairn_gemm_desc& d, Stream) noexcept {
    if(d.version != 1u && d.version != CAIRN_GEMM_DESC_VERSION) trap();
    const std::size_t lda = d.lda ? d.lda : (d.trans_a ? d.m : d.k), ldb = d.ldb ? d.ldb : (d.trans_b ? d.k : d.n);
    const std::size_t ldc = d.ldc ? d.ldc : d.n;
    for(std::size_t i = 0; i < d.m; ++i)
      for(std::size_t j = 0; j < d.n; ++j) {
        float v;
        if(d.ab_type == CAIRN_TYPE_I8) {
          std::int32_t acc = 0;
          for(std::size_t p = 0; p < d.k; ++p)
            acc += std::int32_t(operand<std::int8_t>(d.a, d.trans_a, i, p, lda)) *
                   std::int32_t(operand<std::int8_t>(d.b, d.trans_b, p, j, ldb));
          if(d.c_type == CAIRN_TYPE_I32) {
            static_cast<std::int32_t*>(d.c)[i * ldc + j] = acc;
            continue;
          }
          v = float(acc);
        } else {
          v = 0.0f;
          for(std::size_t p = 0; p < d.k; ++p) v = v + value(d, d.a, d.trans_a, i, p, lda) * value(d, d.b, d.trans_b, p, j, ldb);
        }
        if(d.row_scale) v = v * d.row_scale[i];
        if(d.col_scale) v = v * d.col_scale[j];
        if(d.bias)
          v = v + (d.bias_type == CAIRN_TYPE_BF16 ? float(static_cast<const cr::bf16*>(d.bias)[j])
                                                  : static_cast<const float*>(d.bias)[j]);
        if(d.act == CAIRN_ACT_RELU) v = v < 0.0f ? 0.0f : v;
        else if(d.act == CAIRN_ACT_GELU) v = float(0.5 * double(v) * (1.0 + std::erf(double(v) / std::sqrt(2.0))));
        if(d.c_type == CAIRN_TYPE_F32) {
          float* out = static_cast<float*>(d.c) + i * ldc + j;
          *out = d.accumulate ? *out + v : v;
        } else if(d.c_type == CAIRN_TYPE_BF16) {
          static_cast<cr::bf16*>(d.c)[i * ldc + j] = fp::narrow<cr::bf16>(double(v));
        } else if(d.c_type == CAIRN_TYPE_F16) {
          static_cast<cr::f16*>(d.c)[i * ldc + j] = fp::narrow<cr::f16>(double(v));
        } else {
          trap();
        }
      }
  }
  template<class T> static T operand(const void* p, int trans, std::size_t r, std::size_t c, std::size_t ld) noexcept {
    return static_cast<const T*>(p)[trans ? c * ld + r : r * ld + c];
  }
  static float value(const cairn_gemm_desc& d, const void* p, int trans, std::size_t r, std::size_t c,
                     std::size_t ld) noexcept {
    switch(d.ab_type) {
      case CAIRN_TYPE_F16: return float(operand<cr::f16>(p, trans, r, c, ld));
      case CAIRN_TYPE_BF16: return float(operand<cr::bf16>(p, trans, r, c, ld));
      case CAIRN_TYPE_F8E4M3: return float(operand<cr::f8e4m3>(p, trans, r, c, ld));
      case CAIRN_TYPE_F8E5M2: return float(operand<cr::f8e5m2>(p, trans, r, c, ld));
      default: trap();
    }
  }
};

using Machine = Emulated;

}  // namespace cr::gpu
