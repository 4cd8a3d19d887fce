// Storage floats: cr::f16, cr::bf16, cr::f8e4m3 and cr::f8e5m2 hold a pattern and convert; they never compute. The
// names, layouts and conversion rules are CAIRN's (src/cairn/runtime/cairn_float.hpp:11-175, docs/numerics.md
// "Storage floats"): IEEE 754 binary16 and bfloat16, OCP E4M3 (no infinity, largest 448) and E5M2. Widening is exact;
// narrow<T>(x) rounds once to nearest, ties to even, gives infinity past the largest finite value (E4M3, which has
// none, traps there) and turns a NaN into the format's quiet NaN with x's sign; quantize<T>(x, scale) rounds
// x / scale (exact in double) once and saturates at T's finite range, an integer T included.
//
// The rounding here is integer arithmetic on the double's fields: the significand shifted down to the target's
// spacing, the dropped bits compared with half a unit.
#pragma once
#include <cstdint>
#include <limits>
#include <type_traits>
#include "cairn_runtime.hpp"

namespace cr {
namespace fp {

CR_HD inline std::uint64_t bits_of(double x) noexcept { return __builtin_bit_cast(std::uint64_t, x); }
CR_HD inline double double_of(std::uint64_t u) noexcept { return __builtin_bit_cast(double, u); }

template<int E, int M, bool INF> struct Float {
  using Bits = std::conditional_t<(1 + E + M > 8), std::uint16_t, std::uint8_t>;
  static constexpr int exponent = E, fraction = M;
  static constexpr bool infinite = INF;
  static constexpr int bias = (1 << (E - 1)) - 1;
  static constexpr unsigned top = (1u << E) - 1, ones = (1u << M) - 1;
  static constexpr Bits sign = Bits(1u << (E + M));
  static constexpr Bits nan = Bits(INF ? (top << M) | (1u << (M - 1)) : (top << M) | ones);
  static constexpr Bits largest = Bits(INF ? ((top - 1) << M) | ones : (top << M) | (ones - 1));
  static constexpr Bits infinity = Bits(top << M);
  Bits bits;

  // The value, exactly: every value of these formats is a double.
  explicit operator double() const noexcept {
    const std::uint64_t s = std::uint64_t(bits >> (E + M)) << 63;
    const unsigned e = (bits >> M) & top;
    std::uint64_t f = bits & ones;
    if(e == top && (INF || f == ones))
      return double_of(s | 0x7ff0000000000000ULL | (f ? (1ULL << 51) | (f << (52 - M)) : 0));
    int ex = int(e) - bias;
    if(e == 0) {  // f * 2^(1 - bias - M): normalize into the double's significand
      if(!f) return double_of(s);
      ex = 1 - bias;
      while(!(f >> M)) f <<= 1, --ex;
      f &= ones;
    }
    return double_of(s | (std::uint64_t(ex + 1023) << 52) | (f << (52 - M)));
  }
  explicit operator float() const noexcept { return float(double(*this)); }
};

// |x| (finite, not NaN) rounded to T's grid with its exponent unbounded above, ties to even; `over` says the
// result passes T's largest finite value. Returns the pattern without its sign. Host and device: the device
// quantize kernel takes this path wherever its f32 shortcut cannot decide.
template<class T> CR_HD inline typename T::Bits round_magnitude(double x, bool& over) noexcept {
  constexpr int M = T::fraction, emin = 1 - T::bias;
  const std::uint64_t u = bits_of(x) & 0x7fffffffffffffffULL;
  over = false;
  const int field = int(u >> 52);
  if(field == 0) return 0;  // zero or a double subnormal: below half of every format's least subnormal
  const std::uint64_t sig = (u & ((1ULL << 52) - 1)) | (1ULL << 52);
  const int ex = field - 1023;                  // |x| = sig * 2^(ex - 52)
  const int spacing = (ex < emin ? emin : ex) - M;  // the grid: multiples of 2^spacing
  const int drop = spacing - (ex - 52);         // bits of sig below the grid, > 0 for every format here
  std::uint64_t n;
  if(drop >= 64) n = 0;
  else {
    n = sig >> drop;
    const std::uint64_t rest = sig & ((1ULL << drop) - 1), half = 1ULL << (drop - 1);
    if(rest > half || (rest == half && (n & 1))) ++n;
  }
  // n units of 2^spacing. Below the normal range the pattern is n itself (n == 2^M is the least normal).
  if(ex < emin) return typename T::Bits(n);
  int e = ex;
  if(n >> (M + 1)) n >>= 1, ++e;  // the rounding carried into the next binade
  const unsigned biased = unsigned(e + T::bias);
  const unsigned frac = unsigned(n) & T::ones;
  if(biased > T::top || (biased == T::top && (T::infinite || frac == T::ones))) {
    over = true;
    return 0;
  }
  return typename T::Bits((biased << M) | frac);
}

template<class T> inline T narrow(double x) noexcept {
  const typename T::Bits s = (bits_of(x) >> 63) ? T::sign : typename T::Bits(0);
  if(x != x) return T{typename T::Bits(s | T::nan)};
  bool over = false;
  const typename T::Bits b = (bits_of(x) & 0x7fffffffffffffffULL) == 0x7ff0000000000000ULL ? (over = true, 0)
                                                                                            : round_magnitude<T>(x, over);
  if(over) {
    if constexpr(!T::infinite) trap();
    return T{typename T::Bits(s | T::infinity)};
  }
  return T{typename T::Bits(s | b)};
}

template<class T> inline T quantize(float x, float scale) noexcept {
  if(!(scale > 0.0f) || !(scale <= std::numeric_limits<float>::max())) trap();
  const double q = double(x) / double(scale);
  if constexpr(std::is_integral_v<T>) {
    if(q != q) trap();
    if(q <= double(std::numeric_limits<T>::min())) return std::numeric_limits<T>::min();
    if(q >= double(std::numeric_limits<T>::max())) return std::numeric_limits<T>::max();
    const double a = q < 0 ? -q : q;
    std::int64_t w = std::int64_t(a);
    const double rest = a - double(w);
    if(rest > 0.5 || (rest == 0.5 && (w & 1))) ++w;
    return T(q < 0 ? -w : w);
  } else {
    const typename T::Bits s = (bits_of(q) >> 63) ? T::sign : typename T::Bits(0);
    if(q != q) return T{typename T::Bits(s | T::nan)};
    bool over = false;
    const typename T::Bits b = (bits_of(q) & 0x7fffffffffffffffULL) == 0x7ff0000000000000ULL
                                   ? (over = true, 0)
                                   : round_magnitude<T>(q, over);
    return T{typename T::Bits(s | (over ? T::largest : b))};
  }
}

}  // namespace fp

using f16 = fp::Float<5, 10, true>;
using bf16 = fp::Float<8, 7, true>;
using f8e4m3 = fp::Float<4, 3, false>;
using f8e5m2 = fp::Float<5, 2, true>;
static_assert(sizeof(f16) == 2 && sizeof(bf16) == 2 && sizeof(f8e4m3) == 1 && sizeof(f8e5m2) == 1);
static_assert(std::is_trivially_copyable_v<bf16> && std::is_standard_layout_v<f8e4m3>);

}  // namespace cr
