// The device quantize's element arithmetic (cairn_amd/csrc/quantize.hpp), compiled for the host, against the
// oracle's restatement of the reference's quantize (oracle/oracle.c, src/cairn/runtime/cairn_float.hpp:116-146).
//
// The kernel decides most elements with an f32 shortcut and sends the rest to the reference's double steps; this
// program drives both through the places they can disagree: exact ties, quotients a few units away from every
// rounding boundary of int8 and of both 8-bit floats, the saturation edges, subnormal quotients, the scales at the
// ends of the shortcut's range, and special values. Every answer must equal the oracle's, and the shortcut must
// have both decided and declined on each boundary family (or the boundaries were never reached).
//
// The 8-bit floats' device path (convert_f8) runs here too, on an emulation of the hardware's conversion; it must
// both decide and pass elements on.
//
// Output: one line "checked N decided D declined E converted C passed_on P" and exit 0, or the first mismatch and
// exit 1.
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <random>
#include <vector>
#include "quantize.hpp"

extern "C" {
uint32_t oracle_quantize_float(int f, float x, float scale, int* trapped);
int64_t oracle_quantize_int(float x, float scale, int64_t lo, int64_t hi, int* trapped);
double oracle_decode(int f, uint32_t bits);
}

namespace {

using namespace cairn::quant;
long checked = 0, decided = 0, declined = 0, converted = 0, passed_on = 0;

float bits_f(std::uint32_t u) { return __builtin_bit_cast(float, u); }
std::uint32_t f_bits(float x) { return __builtin_bit_cast(std::uint32_t, x); }

[[noreturn]] void fail(const char* what, float x, float s, long got, long want) {
  std::printf("MISMATCH %s x=%a (0x%08x) s=%a got=%ld want=%ld\n", what, x, f_bits(x), s, got, want);
  std::exit(1);
}

void check_i8(float x, float s) {
  if(!scale_ok(s)) return;
  int t = 0;
  const long want = long(oracle_quantize_int(x, s, -128, 127, &t));
  const float r = 1.0f / s;
  if(fast_ok(s)) {
    int v = 0;
    if(try_i8(x * r, v)) {
      ++decided;
      if(v != want || t) fail("i8 shortcut", x, s, v, t ? -999 : want);
    } else {
      ++declined;
    }
  }
  bool trapped = false;
  const int got = fast_ok(s) && x == x ? fast_i8(x, s, r) : exact_i8(x, s, trapped);
  if(trapped != bool(t) || (!t && got != want)) fail("i8", x, s, trapped ? -999 : got, t ? -999 : want);
  if(x == x) {  // the exact path alone, at every scale
    bool dummy = false;
    const int e = exact_i8(x, s, dummy);
    if(e != want) fail("i8 exact", x, s, e, want);
  }
  ++checked;
}

// The hardware's f32 -> 8-bit float conversion as the device kernel uses it (v_cvt_pk_fp8_f32 / v_cvt_pk_bf8_f32 on
// gfx950, observed on the GPU): OCP formats, round to nearest even with subnormals, no saturation. Below the midpoint
// past the largest value that is the reference's rounding of y itself (scale 1, where saturation and rounding
// agree); at or past it NaN (E4M3) or infinity (E5M2), NaN for a NaN. Its inverse (v_cvt_f32_fp8 / v_cvt_f32_bf8) is
// exact: the oracle's decode.
std::uint32_t conversion(int fmt, float y) {
  const std::uint32_t u = f_bits(y), sign = u >> 31 << 7;
  const std::uint32_t limit = fmt == 3 ? 0x43e80000u : 0x47700000u;  // 464, 61440
  if((u & 0x7fffffffu) > 0x7f800000u) return sign | (fmt == 3 ? 0x7fu : 0x7eu);
  if((u & 0x7fffffffu) >= limit) return sign | (fmt == 3 ? 0x7fu : 0x7cu);
  int t = 0;
  return oracle_quantize_float(fmt, y, 1.0f, &t);
}

template<class T> void check_f8(int fmt, float x, float s) {
  if(!scale_ok(s)) return;
  int t = 0;
  const long want = long(oracle_quantize_float(fmt, x, s, &t));
  const float r = 1.0f / s;
  if(fast_ok_f8(s)) {
    std::uint32_t v = 0;
    if(try_f8<T>(x, x * r, v)) {
      ++decided;
      if(long(v) != want) fail(fmt == 3 ? "e4m3 shortcut" : "e5m2 shortcut", x, s, long(v), want);
    } else {
      ++declined;
    }
  }
  const std::uint32_t got = fast_ok_f8(s) ? fast_f8<T>(x, s, r) : exact_f8<T>(x, s);
  if(long(got) != want) fail(fmt == 3 ? "e4m3" : "e5m2", x, s, long(got), want);
  if(long(exact_f8<T>(x, s)) != want) fail("f8 exact", x, s, long(exact_f8<T>(x, s)), want);
  if(fast_ok_f8(s)) {  // the device kernel's path: convert_f8 on a chunk of eight copies of the element
    float xs[8], y[8];
    for(int e = 0; e < 8; ++e) {
      xs[e] = x;
      y[e] = x * r;
    }
    std::uint32_t o[2] = {};
    const auto word = [&](float a, float b, float c, float d) {
      return conversion(fmt, a) | conversion(fmt, b) << 8 | conversion(fmt, c) << 16 | conversion(fmt, d) << 24;
    };
    const auto decode = [&](std::uint32_t code) { return float(oracle_decode(fmt, code)); };
    if(convert_f8<T>(xs, y, s, o, word, decode)) {
      ++converted;
      if(long(o[0] & 0xffu) != want || o[0] != o[1] || (o[0] & 0xffu) * 0x01010101u != o[0])
        fail(fmt == 3 ? "e4m3 conversion" : "e5m2 conversion", x, s, long(o[0] & 0xffu), want);
    } else {
      ++passed_on;
    }
  }
  ++checked;
}

// x's nearest floats around a target value t (t * s computed in double, then rounded): the tie itself where it is
// representable, and up to `spread` units either side.
template<class F> void around(double target, float s, int spread, F&& f) {
  const float c = float(target * double(s));
  if(!std::isfinite(c)) return;
  const std::uint32_t u = f_bits(c);
  for(int d = -spread; d <= spread; ++d) {
    const std::int64_t w = std::int64_t(u & 0x7fffffffu) + d;
    if(w < 0 || w >= 0x7f800000) continue;
    f(bits_f(std::uint32_t(w) | (u & 0x80000000u)));
  }
}

}  // namespace

int main() {
  std::mt19937_64 rng(20251201);
  std::vector<float> scales = {1.0f, 0.5f, 3.0f, 0.1f, 1.0f / 3.0f, 7.8125e-3f, 1e-3f, 2.5e-2f, 1e-30f, 1e30f,
                               0x1p-120f, 0x1.fffffep-121f, 0x1p120f, 0x1.000002p120f, 0x1p-100f, 0x1.fffffep-101f,
                               0x1p100f, 0x1.000002p100f, 0x1.8p-99f, 0x1.8p99f, 1e-40f, 3e38f, 123.456f};
  std::uniform_real_distribution<double> logu(-40.0, 40.0);
  for(int i = 0; i < 48; ++i) scales.push_back(float(std::pow(2.0, logu(rng))) * float(1.0 + (rng() % 1000) / 997.0));
  // Scales as the kernel computes them: a row's largest magnitude over the format's range.
  for(int i = 0; i < 24; ++i) {
    const float top = float(std::ldexp(1.0 + double(rng() % 8388608) / 8388608.0, int(rng() % 40) - 20));
    scales.push_back(top / 127.0f);
    scales.push_back(top / 448.0f);
    scales.push_back(top / 57344.0f);
  }
  const float specials[] = {0.0f, -0.0f, INFINITY, -INFINITY, NAN, -NAN, 1e-45f, -1e-45f, 1.17549435e-38f,
                            3.40282347e38f, -3.40282347e38f, 1.0f, -1.0f};

  // int8: every half-integer from -130.5 to 130.5 and the saturation edges, a few units around, at every scale.
  long i8_before = declined;
  for(const float s : scales) {
    for(int n = -131; n <= 131; ++n) around(n + 0.5, s, 24, [&](float x) { check_i8(x, s); });
    for(const double e : {127.0, -128.0, 255.9, 256.0, -256.0, 1e6, -1e6})
      around(e, s, 8, [&](float x) { check_i8(x, s); });
    for(const float x : specials) check_i8(x, s);
    std::uniform_real_distribution<float> u(-300.0f, 300.0f);
    for(int i = 0; i < 4000; ++i) check_i8(u(rng) * s, s);
    for(int i = 0; i < 2000; ++i) check_i8(bits_f(std::uint32_t(rng())), s);  // every bit pattern, NaNs included
  }
  if(declined == i8_before) {
    std::printf("int8 ties never reached the exact path\n");
    return 1;
  }

  // 8-bit floats: the midpoint between every pair of neighbouring values (and 0 and the least subnormal), the
  // values themselves, and the saturation edge, a few units around, at every scale.
  auto floats = [&](int fmt, auto tag) {
    using T = decltype(tag);
    const int count = 128;  // the magnitudes: patterns 0 .. 127
    std::vector<double> values;
    for(int p = 0; p < count; ++p) {
      const double v = oracle_decode(fmt, std::uint32_t(p));
      if(std::isfinite(v)) values.push_back(v);
    }
    const double top = values.back();
    const long before = declined;
    for(const float s : scales) {
      for(std::size_t i = 0; i + 1 < values.size(); ++i) {
        const double mid = 0.5 * (values[i] + values[i + 1]);
        for(const double sign : {1.0, -1.0}) {
          around(sign * mid, s, 20, [&](float x) { check_f8<T>(fmt, x, s); });
          around(sign * values[i + 1], s, 4, [&](float x) { check_f8<T>(fmt, x, s); });
        }
      }
      const double step = values.back() - values[values.size() - 2];
      for(const double e : {top + step / 2, top + step, 2 * top, 1e9})
        for(const double sign : {1.0, -1.0}) around(sign * e, s, 8, [&](float x) { check_f8<T>(fmt, x, s); });
      for(const float x : specials) check_f8<T>(fmt, x, s);
      std::uniform_real_distribution<float> u(float(-1.2 * top), float(1.2 * top));
      for(int i = 0; i < 3000; ++i) check_f8<T>(fmt, u(rng) * s, s);
      for(int i = 0; i < 2000; ++i) check_f8<T>(fmt, bits_f(std::uint32_t(rng())), s);
    }
    if(declined == before) {
      std::printf("format %d midpoints never reached the exact path\n", fmt);
      std::exit(1);
    }
  };
  floats(3, cr::f8e4m3{});
  floats(4, cr::f8e5m2{});
  if(converted == 0 || passed_on == 0) {
    std::printf("the conversion path never %s\n", converted ? "passed an element on" : "decided");
    return 1;
  }
  std::printf("checked %ld decided %ld declined %ld converted %ld passed_on %ld\n", checked, decided, declined,
              converted, passed_on);
  return 0;
}
