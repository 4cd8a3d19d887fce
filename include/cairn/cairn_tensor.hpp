// The tensor-core multiply's C++20 entry points, with the spellings CAIRN-emitted code calls
// (src/cairn/compiler/device/tensor.py:69-82): cr::tensor::multiply<A> on host views and
// cr::tensor::launch<A>(cr::gpu::here(), ...) on device views. mma_unordered(m, n, k, c, a, b) adds the product of
// the row-major m x k matrix a and the row-major k x n matrix b, both of one storage float, into the row-major m x n
// f32 matrix c, under the contract of docs/numerics.md: exact products, f32 sums in an order the hardware picks,
// within (k + 1) * 2^-22 * (|c| + sum |a * b|) of the exact sum.
//
// On the host the multiply is its own reference: for each output its old value, then its products in increasing p,
// every step an f32 rounding (src/cairn/runtime/cairn_tensor.hpp:26-41). On the device it is one call to the machine
// the context runs on: the HIP machine queues the gfx950 MFMA kernels of libcairn_gemm_gfx950.so through its C ABI.
// cr::tensor::gemm is the same on a cairn_gemm_desc: layouts, epilogues and int8 beyond what mma_unordered says.
#pragma once
#include <cstddef>
#include <type_traits>
#include "../cairn_gemm.h"
#include "cairn_context.hpp"
#include "cairn_float.hpp"

namespace cr::tensor {

// The extents agree with the views: c holds m * n, a holds m * k and b holds k * n elements.
inline void shape(std::size_t m, std::size_t n, std::size_t k, std::size_t c, std::size_t a, std::size_t b) noexcept {
  if(cr::mul(m, n) != c || cr::mul(m, k) != a || cr::mul(k, n) != b) trap();
}

// The host loop: rows outermost, then p upward, then along a row of b and c, so each output sees its products in
// increasing p. Built without FMA contraction (-ffp-contract=off), so each product and each sum rounds alone.
template<class A> inline void reference(std::size_t m, std::size_t n, std::size_t k, float* c, const A* a,
                                        const A* b) noexcept {
  for(std::size_t i = 0; i < m; ++i) {
    float* row = c + i * n;
    for(std::size_t p = 0; p < k; ++p) {
      const float x = static_cast<float>(a[i * k + p]);
      const A* brow = b + p * n;
      for(std::size_t j = 0; j < n; ++j) row[j] = row[j] + x * static_cast<float>(brow[j]);
    }
  }
}

template<class A> inline void multiply(std::size_t m, std::size_t n, std::size_t k, float* c, std::size_t cn,
                                       const A* a, std::size_t an, const A* b, std::size_t bn) noexcept {
  shape(m, n, k, cn, an, bn);
  reference(m, n, k, c, a, b);
}

// The C ABI's name for a storage float.
template<class A> constexpr int type_of() noexcept {
  if constexpr(std::is_same_v<A, cr::f16>) return CAIRN_TYPE_F16;
  else if constexpr(std::is_same_v<A, cr::bf16>) return CAIRN_TYPE_BF16;
  else if constexpr(std::is_same_v<A, cr::f8e4m3>) return CAIRN_TYPE_F8E4M3;
  else if constexpr(std::is_same_v<A, cr::f8e5m2>) return CAIRN_TYPE_F8E5M2;
  else static_assert(sizeof(A) == 0, "mma_unordered multiplies storage floats");
}

// On the calling thread's execution context: the multiply runs as its synchronous work and the call returns once that
// stream has run it (in a held run, at the run's end; under an enqueued call, never). m or n of 0 queues nothing,
// and so does k of 0, which leaves c as it is.
template<class A, class M>
inline void launch(reuse::Context<M>& ctx, std::size_t m, std::size_t n, std::size_t k, float* c, std::size_t cn,
                   const A* a, std::size_t an, const A* b, std::size_t bn) noexcept {
  shape(m, n, k, cn, an, bn);
  if(!m || !n || !k) return;
  reuse::synchronous(ctx, [&](typename M::Stream s) { ctx.machine().mma(type_of<A>(), m, n, k, c, a, b, s); });
}

// Any GEMM the C ABI describes, as synchronous work on the context.
template<class M> inline void gemm(reuse::Context<M>& ctx, const cairn_gemm_desc& d) noexcept {
  reuse::synchronous(ctx, [&](typename M::Stream s) { ctx.machine().gemm(d, s); });
}

}  // namespace cr::tensor
