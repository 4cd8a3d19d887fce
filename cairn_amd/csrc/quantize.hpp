// One element of quantize[T](x, scale) (src/cairn/runtime/cairn_float.hpp:116-146): x / scale, the quotient taken
// in double, rounded once to nearest with ties to even and saturated at T's finite range. T here is int8 (the W8A8
// operand) or one of the 8-bit floats (E4M3, E5M2).
//
// The double quotient is exact to far better than the rounding needs, but a double division per element costs more
// than HBM allows a bandwidth-bound kernel, so each element first takes an f32 shortcut and falls back to the double
// path only where the shortcut cannot decide:
//
//   r = 1 / scale rounded to f32 (once per row) and y = x * r rounded to f32 give |y - q| <= |q| * 2^-22 for the
//   exact q = x / scale, as long as scale lies in [2^-120, 2^120] (so r is a normal float and x * r overflows only
//   where q saturates anyway). Where y is farther than that from every rounding boundary of T (the half-integers for
//   int8, the midpoints between neighbours of T's grid for the floats) q rounds to the same value as y, and no tie
//   is possible; otherwise the element takes the exact double path.
//
// Both paths compile for the host too, so a CPU test drives the shortcut through every boundary and compares it with
// the reference's formula. Where the reference traps (a scale that is not positive and finite, a NaN quantized to an
// integer) these functions report it through `trapped` and return 0: a kernel cannot abort.
#pragma once
#include <cstdint>
#include "../../include/cairn/cairn_float.hpp"

namespace cairn::quant {

constexpr float FAST_LO = 0x1p-120f, FAST_HI = 0x1p120f;

// Whether a scale is one the reference accepts: positive and finite.
CR_HD inline bool scale_ok(float s) { return s > 0.0f && s <= 3.40282347e38f; }
// Whether the f32 shortcut is sound for this scale (a property of the row, so the branch is uniform).
CR_HD inline bool fast_ok(float s) { return s >= FAST_LO && s <= FAST_HI; }

// int8, exactly the reference's steps: the double quotient, saturation, then ties to even on its magnitude.
CR_HD inline int exact_i8(float x, float s, bool& trapped) {
  const double q = double(x) / double(s);
  if(q != q) {
    trapped = true;
    return 0;
  }
  if(q <= -128.0) return -128;
  if(q >= 127.0) return 127;
  const double a = q < 0 ? -q : q;
  int w = int(a);                      // a < 128: the truncation is exact
  const double rest = a - double(w);   // exact: a and w share a binade or w is 0
  if(rest > 0.5 || (rest == 0.5 && (w & 1))) ++w;
  return q < 0 ? -w : w;
}

// y = x * r within 2^-22 |q| of q and |y| < 256 put q within 2^-14 of y; a y 2^-13 or more from the half-integers
// about it therefore rounds as q does. |y| >= 256 means |q| > 255: saturated either way. Returns whether y decided.
CR_HD inline bool try_i8(float y, int& out) {
  if(__builtin_fabsf(y) >= 256.0f) {
    out = y < 0.0f ? -128 : 127;
    return true;
  }
  const float n = __builtin_rintf(y);                       // ties to even, as the exact path's
  const bool ok = __builtin_fabsf(y - n) <= 0.5f - 0x1p-13f;  // the difference is exact; false for a NaN y
  const int v = int(ok ? n : 0.0f);
  out = v < -128 ? -128 : (v > 127 ? 127 : v);
  return ok;
}

CR_HD inline int fast_i8(float x, float s, float r, bool& trapped) {
  int v;
  return try_i8(x * r, v) ? v : exact_i8(x, s, trapped);
}

// An 8-bit float (cr::f8e4m3 or cr::f8e5m2), exactly the reference's steps: the double quotient, its sign (x's, as
// scale > 0; also for a NaN), NaN to the format's NaN, everything past the largest finite value to the largest.
template<class T> CR_HD inline std::uint32_t exact_f8(float x, float s) {
  const double q = double(x) / double(s);
  const std::uint32_t sign = (__builtin_bit_cast(std::uint32_t, x) >> 31) ? T::sign : 0u;
  if(x != x) return sign | T::nan;
  const double a = q < 0 ? -q : q;
  if(a > 1.7976931348623157e308) return sign | T::largest;  // an infinite x
  bool over = false;
  const std::uint32_t b = cr::fp::round_magnitude<T>(a, over);
  return sign | (over ? std::uint32_t(T::largest) : b);
}

// The shortcut on y = x * r's own bits: |y| = sig * 2^(e - 23) with a 24-bit sig; T's grid at y is multiples of
// 2^spacing, so `drop` low bits of sig fall below it and the boundary is where they equal half a unit. |y - q| is
// under 4.01 units of y's last place (|q| < 2^(e+1) (1 + 2^-22), times 2^-22), so a boundary more than 8 units away
// is on the same side for y and q. The carry into the next binade and the saturation are the exact path's rules.
// Returns whether y decided; `out` holds y's rounding either way.
template<class T> CR_HD inline bool try_f8(float x, float y, std::uint32_t& out) {
  constexpr int M = T::fraction, emin = 1 - T::bias;
  constexpr std::uint32_t TOL = 8;
  const std::uint32_t u = __builtin_bit_cast(std::uint32_t, y);
  const std::uint32_t sign = (__builtin_bit_cast(std::uint32_t, x) >> 31) ? T::sign : 0u;
  const std::uint32_t mag = u & 0x7fffffffu;
  out = sign;
  if(mag > 0x7f800000u) return out |= T::nan, true;       // x is a NaN (r is finite and positive)
  if(mag == 0x7f800000u) return out |= T::largest, true;  // x infinite, or q far past the largest value
  const int field = int(mag >> 23);
  if(field == 0) return true;  // |y| < 2^-126: q is far below half of T's least subnormal
  const int e = field - 127;
  const std::uint32_t sig = (mag & 0x7fffffu) | 0x800000u;
  const int drop = 23 - M + (e < emin ? emin - e : 0);
  if(drop > 26) return true;  // half a unit of T's grid exceeds 4 |y|
  const std::uint32_t rest = sig & ((1u << drop) - 1u), half = 1u << (drop - 1);
  const std::uint32_t dist = rest > half ? rest - half : half - rest;
  std::uint32_t n = (sig >> drop) + (rest > half ? 1u : 0u);
  if(e < emin) {
    out |= n;  // subnormal (n == 2^M is the least normal, whose pattern is n)
  } else {
    int biased = e + T::bias;
    if(n >> (M + 1)) {
      n >>= 1;
      ++biased;
    }
    const std::uint32_t frac = n & T::ones;
    const bool over = biased > int(T::top) || (biased == int(T::top) && (T::infinite || frac == T::ones));
    out |= over ? std::uint32_t(T::largest) : (std::uint32_t(biased) << M) | frac;
  }
  return dist > TOL;
}

template<class T> CR_HD inline std::uint32_t fast_f8(float x, float s, float r) {
  std::uint32_t v;
  return try_f8<T>(x, x * r, v) ? v : exact_f8<T>(x, s);
}

// The divisor the per-row scale is taken against: T's largest finite magnitude.
template<class T> constexpr float range_of() {
  if constexpr(sizeof(T) == 1 && std::is_integral_v<T>) return 127.0f;
  else return T::infinite ? 57344.0f : 448.0f;
}

}  // namespace cairn::quant
