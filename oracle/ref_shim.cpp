// TEST INFRASTRUCTURE ONLY: C linkage over the reference's own header-only host multiply and storage floats, so
// the oracle can be checked against the reference's bits. The reference headers are read where they lie
// (REF_RUNTIME=/root/reference/src/cairn/runtime); nothing of them is copied into this repository. The library this
// builds goes to oracle/_ref/ only, and is used by tests/golden/make_golden.py (fixtures) and bench.py's
// cpu_baseline leg (the reference loop timed on the host).
//
//   ref_mma_*       cr::tensor::multiply<A>   cairn_tensor.hpp:37-41
//   ref_decode_*    Float::operator double    cairn_float.hpp:35-48
//   ref_narrow_*    cr::fp::narrow<T>         cairn_float.hpp:100-110
//   ref_quantize_*  cr::fp::quantize<T>       cairn_float.hpp:116-146
#include <cstddef>
#include <cstdint>
#include "cairn_tensor.hpp"

#define CAIRN_REF_FORMAT(NAME, T, BITS)                                                                           \
  extern "C" void ref_mma_##NAME(std::size_t m, std::size_t n, std::size_t k, float* c, std::size_t cn,         \
                                 const BITS* a, std::size_t an, const BITS* b, std::size_t bn) {                 \
    static_assert(sizeof(T) == sizeof(BITS));                                                                     \
    cr::tensor::multiply<T>(m, n, k, c, cn, reinterpret_cast<const T*>(a), an, reinterpret_cast<const T*>(b),   \
                            bn);                                                                                  \
  }                                                                                                               \
  extern "C" double ref_decode_##NAME(BITS bits) { return static_cast<double>(T{bits}); }                       \
  extern "C" BITS ref_narrow_##NAME(double x) { return cr::fp::narrow<T>(x).bits; }                             \
  extern "C" BITS ref_quantize_##NAME(float x, float scale) { return cr::fp::quantize<T>(x, scale).bits; }

CAIRN_REF_FORMAT(f16, cr::f16, std::uint16_t)
CAIRN_REF_FORMAT(bf16, cr::bf16, std::uint16_t)
CAIRN_REF_FORMAT(f8e4m3, cr::f8e4m3, std::uint8_t)
CAIRN_REF_FORMAT(f8e5m2, cr::f8e5m2, std::uint8_t)

extern "C" void ref_mma_f32(std::size_t m, std::size_t n, std::size_t k, float* c, std::size_t cn, const float* a,
                            std::size_t an, const float* b, std::size_t bn) {
  cr::tensor::multiply<float>(m, n, k, c, cn, a, an, b, bn);
}
extern "C" std::int8_t ref_quantize_i8(float x, float scale) { return cr::fp::quantize<std::int8_t>(x, scale); }
