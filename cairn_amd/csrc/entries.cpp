// The multiply's CAIRN entries (include/cairn_gemm.h, layer 1): what CAIRN's compiler emits around a function whose
// body is mma_unordered(m, n, k, c, a, b) (tests/soundness/test_tensor.py:31-36), for host views and for device
// views, with its checked entry cf_NAME, its enqueued entry cq_NAME and the stream binding
// (src/cairn/compiler/lower/header.py:215-249,283-313; codegen.py:500-512 for the view checks). They are written
// against the C++20 surface (include/cairn/), as emitted code is.
#include <cstddef>
#include "../../include/cairn/cairn_hip.hpp"
#include "../../include/cairn/cairn_here.hpp"
#include "../../include/cairn/cairn_tensor.hpp"

namespace {
// The checked entry's guards: every view valid for its count, and the read-write c sharing no byte with a or b
// (a and b may be one array).
template<class A> void checked(float* c, std::size_t cn, const A* a, std::size_t an, const A* b, std::size_t bn) {
  cr::view(c, cn);
  cr::view(a, an);
  cr::view(b, bn);
  cr::disjoint(c, cn, a, an);
  cr::disjoint(c, cn, b, bn);
}
}  // namespace

#define CAIRN_HOST_ENTRY(NAME, T, C)                                                                              \
  extern "C" __attribute__((visibility("default"))) void cf_mma_##NAME(                                         \
      std::size_t m, std::size_t n, std::size_t k, std::size_t cn, float* c, std::size_t an, const C* a,        \
      std::size_t bn, const C* b) {                                                                      \
    static_assert(sizeof(T) == sizeof(C));                                                                        \
    const T* x = reinterpret_cast<const T*>(a);                                                                   \
    const T* y = reinterpret_cast<const T*>(b);                                                                   \
    checked(c, cn, x, an, y, bn);                                                                                 \
    cr::tensor::multiply<T>(m, n, k, c, cn, x, an, y, bn);                                                        \
  }

#define CAIRN_DEVICE_ENTRY(NAME, T, C)                                                                            \
  extern "C" __attribute__((visibility("default"))) void cf_mma_##NAME##_device(                                \
      std::size_t m, std::size_t n, std::size_t k, std::size_t cn, float* c, std::size_t an, const C* a,        \
      std::size_t bn, const C* b) {                                                                      \
    const T* x = reinterpret_cast<const T*>(a);                                                                   \
    const T* y = reinterpret_cast<const T*>(b);                                                                   \
    checked(c, cn, x, an, y, bn);                                                                                 \
    cr::tensor::launch<T>(cr::gpu::here(), m, n, k, c, cn, x, an, y, bn);                                         \
  }                                                                                                               \
  extern "C" __attribute__((visibility("default"))) void cq_mma_##NAME##_device(                                \
      void* stream, std::size_t m, std::size_t n, std::size_t k, std::size_t cn, float* c, std::size_t an,       \
      const C* a, std::size_t bn, const C* b) {                                                          \
    const cr::gpu::Enqueued on(stream);                                                                           \
    cf_mma_##NAME##_device(m, n, k, cn, c, an, a, bn, b);                                                         \
  }

CAIRN_HOST_ENTRY(f32, float, float)
CAIRN_HOST_ENTRY(f16, cr::f16, cairn_f16)
CAIRN_HOST_ENTRY(bf16, cr::bf16, cairn_bf16)
CAIRN_HOST_ENTRY(f8e4m3, cr::f8e4m3, cairn_f8e4m3)
CAIRN_HOST_ENTRY(f8e5m2, cr::f8e5m2, cairn_f8e5m2)
CAIRN_DEVICE_ENTRY(f16, cr::f16, cairn_f16)
CAIRN_DEVICE_ENTRY(bf16, cr::bf16, cairn_bf16)
CAIRN_DEVICE_ENTRY(f8e4m3, cr::f8e4m3, cairn_f8e4m3)
CAIRN_DEVICE_ENTRY(f8e5m2, cr::f8e5m2, cairn_f8e5m2)

extern "C" __attribute__((visibility("default"))) void cairn_gemm_device_stream(void* stream) {
  cr::gpu::use_stream(stream);
}
