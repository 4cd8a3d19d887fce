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
// about it therefore rounds as q does. |y| >= 256 means |q| > 255: saturated either way, so y is clamped to +-256
// first (an integer: distance 0). round_i8 gives the candidate and y's distance from it, branch-free (every lane of
// a wave runs the same instructions); the candidate is q's answer where that distance is at most MARGIN_I8.
constexpr float MARGIN_I8 = 0.5f - 0x1p-13f;
CR_HD inline int round_i8(float y, float& dev) {
  const float c = __builtin_fminf(__builtin_fmaxf(y, -256.0f), 256.0f);
  const float n = __builtin_rintf(c);  // ties to even, as the exact path's
  dev = __builtin_fabsf(c - n);        // exact: c and n are within a factor of two, or n is 0
  return int(__builtin_fminf(__builtin_fmaxf(n, -128.0f), 127.0f));
}

// Whether y decides: not a NaN (which clamps to a bound and has no int8 answer) and far enough from a tie.
CR_HD inline bool try_i8(float y, int& out) {
  float dev;
  out = round_i8(y, dev);
  return y == y && dev <= MARGIN_I8;
}

// Where round_i8 leaves it, y lies within 2^-13 of a half-integer h and q within 2^-12 of it, so q rounds to the
// integer n nearest y or to its neighbour across h. One fused multiply-add decides which, exactly: x - h * s, rounded
// once, has the sign of q - h and is zero only at a tie (with scale in the shortcut's range every such difference is
// a multiple of 2^-149, which the fma represents; an overflow keeps the sign). A tie goes to the even integer. No
// double arithmetic, and the same answer as the reference's rounding of the double quotient (which is within 2^-37
// of q, and q is either a tie or at least 2^-25 away from one).
CR_HD inline int near_i8(float x, float s, float y) {
  const float c = __builtin_fminf(__builtin_fmaxf(y, -256.0f), 256.0f);
  const float n = __builtin_rintf(c);
  const float step = c > n ? 1.0f : -1.0f;
  const float h = n + 0.5f * step, other = n + step;
  const float e = __builtin_fmaf(-h, s, x);
  const bool even = (int(n) & 1) == 0;
  const float pick = e == 0.0f ? (even ? n : other) : ((e > 0.0f) == (step > 0.0f) ? other : n);
  return int(__builtin_fminf(__builtin_fmaxf(pick, -128.0f), 127.0f));
}

// x (not a NaN) into int8 at a scale in the shortcut's range: the shortcut, else the fma decision.
CR_HD inline int fast_i8(float x, float s, float r) {
  int v;
  const float y = x * r;
  return try_i8(y, v) ? v : near_i8(x, s, y);
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

// Where try_f8 leaves it (y within 8 units of its last place of a midpoint of T's grid), the answer exactly: the
// midpoint is (2 below + 1) * 2^(spacing - 1), `below` being the grid units under it, and |x| - mid * s by one fused
// multiply-add has the sign of |q| - mid and is zero only at a tie (with scale in [2^-100, 2^100] the product stays
// finite and every such difference is a multiple of 2^-149). A tie goes to the even unit; then the encoding of
// try_f8 (the carry into the next binade, subnormals, saturation).
template<class T> CR_HD inline std::uint32_t near_f8(float x, float s, float y) {
  constexpr int M = T::fraction, emin = 1 - T::bias;
  const std::uint32_t mag = __builtin_bit_cast(std::uint32_t, y) & 0x7fffffffu;
  const std::uint32_t sign = (__builtin_bit_cast(std::uint32_t, x) >> 31) ? T::sign : 0u;
  const int e = int(mag >> 23) - 127;
  const std::uint32_t sig = (mag & 0x7fffffu) | 0x800000u;
  const int drop = 23 - M + (e < emin ? emin - e : 0);
  const std::uint32_t below = sig >> drop;
  const float mid = __builtin_ldexpf(float(2u * below + 1u), e - 23 + drop - 1);
  const float d = __builtin_fmaf(-mid, s, __builtin_fabsf(x));
  std::uint32_t n = below + ((d > 0.0f || (d == 0.0f && (below & 1u))) ? 1u : 0u);
  if(e < emin) return sign | n;
  int biased = e + T::bias;
  if(n >> (M + 1)) {
    n >>= 1;
    ++biased;
  }
  const std::uint32_t frac = n & T::ones;
  const bool over = biased > int(T::top) || (biased == int(T::top) && (T::infinite || frac == T::ones));
  return sign | (over ? std::uint32_t(T::largest) : (std::uint32_t(biased) << M) | frac);
}

// The 8-bit floats' shortcut is sound on a narrower range of scales than int8's: the midpoint times the scale must
// stay finite in near_f8.
CR_HD inline bool fast_ok_f8(float s) { return s >= 0x1p-100f && s <= 0x1p100f; }

// Eight elements x into T, given y = x * (1 / s), through a round-to-nearest-even conversion `word` (four f32 to
// four codes in one word, low byte first) that does not saturate, and its exact inverse `decode` (a code's magnitude
// bits to f32). The device passes the hardware's (v_cvt_pk_fp8_f32 / v_cvt_pk_bf8_f32 and v_cvt_f32_fp8 /
// v_cvt_f32_bf8: the OCP formats, ties to even, subnormals kept; past the last midpoint NaN for E4M3, infinity for
// E5M2). Sound for scales where fast_ok_f8 holds.
//
// y is within 2^-23 |y| (relative) of x / s, so x / s lies between y (1 - 2^-21) and y (1 + 2^-21), each rounded to
// f32; rounding is monotonic, so the answer lies between their codes lo and hi. Where lo and hi agree, that is the
// answer. Otherwise they are neighbours (the margin is far below the grid's spacing) and the midpoint between them
// decides, as in near_f8: |x| - mid * s by one fused multiply-add has the sign of |x / s| - mid and is zero only at
// a tie, which goes to the even code.
//
// Returns false, with o unspecified, where an element's |y| is not below LIMIT, the midpoint above the largest
// finite value (464 for E4M3, 61440 for E5M2), or where hi passes the largest value: up to LIMIT nearest-even gives
// the largest value, as the reference's saturation does, but past it (and for a NaN) the conversion's codes are not
// the reference's. The caller then decides the chunk element by element.
template<class T, class Word, class Decode>
CR_HD inline bool convert_f8(const float (&x)[8], const float (&y)[8], float s, std::uint32_t (&o)[2], Word&& word,
                             Decode&& decode) {
  constexpr float DOWN = 0x1.fffff0p-1f, UP = 0x1.000008p+0f;           // 1 - 2^-21, 1 + 2^-21
  constexpr std::uint32_t LIMIT = T::infinite ? 0x47700000u : 0x43e80000u;  // 61440, 464 as f32
  std::uint32_t top = 0;  // the largest |y| pattern: a NaN's orders above every finite value and infinity
  for(int e = 0; e < 8; ++e) {
    const std::uint32_t u = __builtin_bit_cast(std::uint32_t, y[e]) & 0x7fffffffu;
    top = u > top ? u : top;
  }
  if(top >= LIMIT) return false;
  bool ok = true;
  for(int h = 0; h < 2; ++h) {
    const float* v = y + 4 * h;
    const std::uint32_t c = word(v[0], v[1], v[2], v[3]);
    const std::uint32_t lo = word(v[0] * DOWN, v[1] * DOWN, v[2] * DOWN, v[3] * DOWN);
    const std::uint32_t hi = word(v[0] * UP, v[1] * UP, v[2] * UP, v[3] * UP);
    o[h] = c;
    if(lo == hi) continue;  // then c, between them, equals both
    std::uint32_t out = 0;
    for(int e = 0; e < 4; ++e) {
      const std::uint32_t cb = (c >> (8 * e)) & 0xffu, lm = (lo >> (8 * e)) & 0x7fu, hm = (hi >> (8 * e)) & 0x7fu;
      std::uint32_t pick = lm;
      if(lm != hm) {  // y (1 - 2^-21) has the smaller magnitude, whatever the sign
        ok = ok && hm <= std::uint32_t(T::largest);
        const float mid = 0.5f * (decode(lm) + decode(hm));
        const float d = __builtin_fmaf(-mid, s, __builtin_fabsf(x[4 * h + e]));
        pick = d > 0.0f || (d == 0.0f && (lm & 1u)) ? hm : lm;
      }
      out |= ((cb & 0x80u) | pick) << (8 * e);
    }
    o[h] = out;
  }
  return ok;
}

template<class T> CR_HD inline std::uint32_t fast_f8(float x, float s, float r) {
  std::uint32_t v;
  const float y = x * r;
  return try_f8<T>(x, y, v) ? v : near_f8<T>(x, s, y);
}

// The divisor the per-row scale is taken against: T's largest finite magnitude.
template<class T> constexpr float range_of() {
  if constexpr(sizeof(T) == 1 && std::is_integral_v<T>) return 127.0f;
  else return T::infinite ? 57344.0f : 448.0f;
}

}  // namespace cairn::quant
