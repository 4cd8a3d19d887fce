/*
 * TEST INFRASTRUCTURE ONLY. This file is the CPU oracle the parity tests, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg check the HIP library against. Nothing in the product (cairn_amd/, include/) links, loads or
 * calls it; the product path fails loudly when its HIP library is missing instead of falling back to this code.
 *
 * A plain-C restatement of the reference's host multiply and storage floats (SamMausberg/cairn 1.1.0):
 *
 *   oracle_decode      exact decode of a storage-float pattern         src/cairn/runtime/cairn_float.hpp:11-48
 *   oracle_narrow      RNE encode, overflow to infinity / trap for e4m3 src/cairn/runtime/cairn_float.hpp:54-110
 *   oracle_quantize_*  x / scale, RNE once, saturating                  src/cairn/runtime/cairn_float.hpp:116-146
 *   oracle_mma         c[i][j] += sum_p a[i][p] * b[p][j], p increasing,
 *                      every product and sum rounded to f32, no FMA      src/cairn/runtime/cairn_tensor.hpp:28-41
 *   oracle_shape       the extents check (traps -> returns nonzero)     src/cairn/runtime/cairn_tensor.hpp:22-24
 *
 * and the north-star additions, which no reference function defines (pinned by closed forms in tests/):
 *
 *   oracle_gemm_f64    fp64 product of any layout (NN/NT/TN/TT), with sum |a*b| for the contract bound
 *                      (k + 1) * 2^-22 * (|c| + sum |a*b|) of src/cairn/compiler/device/tensor.py:10-12,32
 *   oracle_gemm_i8     int8 x int8 -> int32, exact
 *   oracle_dequant     bf16((f32(acc) * sa[i]) * sb[j]), each step an f32 rounding
 *   oracle_gelu        0.5 x (1 + erf(x / sqrt 2)) in fp64 (the erf form; the reference has no GELU)
 *   oracle_quantize_rows  a matrix quantized row by row with oracle_quantize_* (per-row, per-tensor or computed
 *                      largest-magnitude scales): the device quantize's contract (the reference has no such kernel)
 *
 * Each function is pinned in tests/test_oracle.py: against golden vectors written from the compiled reference
 * header (tests/golden/), against an exact rational model, and against known answers the reference's docs state.
 *
 * Built by oracle/Makefile with -O2 -ffp-contract=off -fno-fast-math, as the reference's host toolchain builds
 * (src/cairn/projects/toolchain.py:29-30): no contraction, so every f32 product and sum rounds on its own.
 */
#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

enum { F16 = 1, BF16 = 2, F8E4M3 = 3, F8E5M2 = 4, F32 = 0 };

typedef struct {
  int e, m, infinite, width;
} format;

static format fmt_of(int f) {
  switch (f) {
    case F16: return (format){5, 10, 1, 16};
    case BF16: return (format){8, 7, 1, 16};
    case F8E4M3: return (format){4, 3, 0, 8};
    case F8E5M2: return (format){5, 2, 1, 8};
    default: return (format){8, 23, 1, 32};
  }
}

/* The value a pattern denotes (IEEE 754 binary16 and bfloat16, OCP E4M3 and E5M2), cairn_float.hpp:35-48. Every
 * value of these formats is a double, so the decode is exact. E4M3 has no infinity: only exponent and fraction all
 * ones is NaN. */
double oracle_decode(int f, uint32_t bits) {
  if (f == F32) {
    float x;
    memcpy(&x, &bits, 4);
    return (double)x;
  }
  const format t = fmt_of(f);
  const int bias = (1 << (t.e - 1)) - 1;
  const uint32_t top = (1u << t.e) - 1, ones = (1u << t.m) - 1;
  const int negative = (bits >> (t.e + t.m)) & 1;
  const uint32_t e = (bits >> t.m) & top, fr = bits & ones;
  double v;
  if (e == top && (t.infinite || fr == ones)) v = fr ? NAN : INFINITY;
  else if (e == 0) v = ldexp((double)fr, 1 - bias - t.m);
  else v = ldexp((double)(fr | (1u << t.m)), (int)e - bias - t.m);
  return negative ? -v : v;
}

/* |x| rounded to the nearest value of the format with the exponent unbounded above, ties to even, as a value; the
 * rounding is done in units of the spacing of |x|'s binade (floored at the subnormal spacing), where rint is exact. */
static double rounded_magnitude(const format t, double ax) {
  const int bias = (1 << (t.e - 1)) - 1, emin = 1 - bias;
  int ex;
  frexp(ax, &ex);          /* ax = f * 2^ex with f in [0.5, 1): the binade is 2^(ex - 1) */
  int binade = ex - 1;
  if (binade < emin) binade = emin;
  const double unit = ldexp(1.0, binade - t.m);
  return rint(ax / unit) * unit; /* division by a power of two is exact; rint rounds to nearest even */
}

static double largest_finite(const format t) {
  const int bias = (1 << (t.e - 1)) - 1;
  const int top = (1 << t.e) - 1;
  if (t.infinite) return ldexp((double)((2u << t.m) - 1), top - 1 - bias - t.m);
  return ldexp((double)((2u << t.m) - 2), top - bias - t.m); /* E4M3: all-ones fraction at the top is NaN */
}

/* The pattern of a finite, non-negative value the format holds. */
static uint32_t encode_magnitude(const format t, double v) {
  const int bias = (1 << (t.e - 1)) - 1, emin = 1 - bias;
  if (v == 0.0) return 0;
  if (v < ldexp(1.0, emin)) return (uint32_t)ldexp(v, t.m - emin); /* subnormal: field 0 */
  int ex;
  frexp(v, &ex);
  const int e = ex - 1;
  const uint32_t frac = (uint32_t)(ldexp(v, t.m - e) - ldexp(1.0, t.m));
  return ((uint32_t)(e + bias) << t.m) | frac;
}

static uint32_t quiet_nan(const format t) {
  const uint32_t top = (1u << t.e) - 1;
  return t.infinite ? (top << t.m) | (1u << (t.m - 1)) : (top << t.m) | ((1u << t.m) - 1);
}

/* narrow<T>(x), cairn_float.hpp:100-110: RNE; past the largest finite value infinity, or for E4M3 a trap (reported
 * through *trapped); a NaN becomes the format's quiet NaN with x's sign. */
uint32_t oracle_narrow(int f, double x, int* trapped) {
  const format t = fmt_of(f);
  const uint32_t sign = signbit(x) ? (1u << (t.e + t.m)) : 0;
  *trapped = 0;
  if (isnan(x)) return sign | quiet_nan(t);
  const double ax = fabs(x);
  const double r = isinf(ax) ? INFINITY : rounded_magnitude(t, ax);
  if (r > largest_finite(t)) {
    if (!t.infinite) {
      *trapped = 1;
      return 0;
    }
    return sign | (((1u << t.e) - 1) << t.m);
  }
  return sign | encode_magnitude(t, r);
}

/* quantize[T](x, scale), cairn_float.hpp:116-146: q = x / scale in double (exact to well within half a unit of
 * every format here), rounded once to nearest even and clamped to T's finite range. A scale that is not positive
 * and finite traps. */
uint32_t oracle_quantize_float(int f, float x, float scale, int* trapped) {
  const format t = fmt_of(f);
  *trapped = !(scale > 0.0f) || !(scale <= 3.4028234663852886e38f);
  if (*trapped) return 0;
  const double q = (double)x / (double)scale;
  const uint32_t sign = signbit(q) ? (1u << (t.e + t.m)) : 0;
  if (isnan(q)) return sign | quiet_nan(t);
  const double aq = fabs(q);
  const double r = isinf(aq) ? INFINITY : rounded_magnitude(t, aq);
  const double top = largest_finite(t);
  return sign | encode_magnitude(t, r > top ? top : r);
}

/* quantize[i8] and the other integers: ties to even, saturating at [lo, hi]; a NaN traps (no integer NaN). */
int64_t oracle_quantize_int(float x, float scale, int64_t lo, int64_t hi, int* trapped) {
  *trapped = !(scale > 0.0f) || !(scale <= 3.4028234663852886e38f) || isnan(x);
  if (*trapped) return 0;
  const double q = (double)x / (double)scale;
  if (q <= (double)lo) return lo;
  if (q >= (double)hi) return hi;
  return (int64_t)rint(q);
}

/* shape(m, n, k, c, a, b), cairn_tensor.hpp:22-24: the extents agree with the views, every product checked for
 * overflow. Returns nonzero where the reference traps. */
int oracle_shape(size_t m, size_t n, size_t k, size_t cn, size_t an, size_t bn) {
  size_t r;
  if (__builtin_mul_overflow(m, n, &r) || r != cn) return 1;
  if (__builtin_mul_overflow(m, k, &r) || r != an) return 1;
  if (__builtin_mul_overflow(k, n, &r) || r != bn) return 1;
  return 0;
}

static float* decode_table(int f) {
  const format t = fmt_of(f);
  const size_t count = (size_t)1 << t.width;
  float* table = malloc(count * sizeof(float));
  for (size_t p = 0; p < count; ++p) table[p] = (float)oracle_decode(f, (uint32_t)p); /* exact: every value is an f32 */
  return table;
}

static uint32_t pattern_at(int f, const void* base, size_t i) {
  if (f == F8E4M3 || f == F8E5M2) return ((const uint8_t*)base)[i];
  return ((const uint16_t*)base)[i];
}

/* reference<A>(m, n, k, c, a, b), cairn_tensor.hpp:28-35: for each row i, each p in increasing order, each column j,
 * c[i][j] = c[i][j] + float(a[i][p]) * float(b[p][j]), every product and every sum an f32 rounding. A is F32 (the
 * template's float instance, config C1) or a storage float decoded exactly. Returns nonzero where shape traps. */
int oracle_mma(int f, size_t m, size_t n, size_t k, float* c, size_t cn, const void* a, size_t an, const void* b,
               size_t bn) {
  if (oracle_shape(m, n, k, cn, an, bn)) return 1;
  if (f == F32) {
    const float* af = a;
    const float* bf = b;
    for (size_t i = 0; i < m; ++i)
      for (size_t p = 0; p < k; ++p) {
        const float x = af[i * k + p];
        for (size_t j = 0; j < n; ++j) c[i * n + j] = c[i * n + j] + x * bf[p * n + j];
      }
    return 0;
  }
  float* table = decode_table(f);
  float* row = malloc((n ? n : 1) * sizeof(float));
  for (size_t i = 0; i < m; ++i)
    for (size_t p = 0; p < k; ++p) {
      const float x = table[pattern_at(f, a, i * k + p)];
      for (size_t j = 0; j < n; ++j) row[j] = table[pattern_at(f, b, p * n + j)];
      for (size_t j = 0; j < n; ++j) c[i * n + j] = c[i * n + j] + x * row[j];
    }
  free(row);
  free(table);
  return 0;
}

/* Element (r, q) of an operand stored row-major with `ld` elements between rows; trans means the stored matrix is
 * the operand's transpose. */
static double element(int f, const void* base, int trans, size_t ld, size_t r, size_t q, const float* table) {
  const size_t at = trans ? q * ld + r : r * ld + q;
  if (f == F32) return ((const float*)base)[at];
  return table[pattern_at(f, base, at)];
}

/* The exact product in fp64 for any layout: out[i][j] = sum_p A[i][p] B[p][j] and mag[i][j] = sum_p |A[i][p] B[p][j]|.
 * A is m x k (trans_a: stored k x m), B is k x n (trans_b: stored n x k). Every product of two 16- or 8-bit floats
 * is exact in fp64; the sums carry fp64's own rounding, far below the f32 contract. */
void oracle_gemm_f64(int f, int trans_a, int trans_b, size_t m, size_t n, size_t k, const void* a, size_t lda,
                     const void* b, size_t ldb, double* out, double* mag) {
  float* table = f == F32 ? NULL : decode_table(f);
  double* bcol = malloc((k ? k : 1) * sizeof(double));
  for (size_t j = 0; j < n; ++j) {
    for (size_t p = 0; p < k; ++p) bcol[p] = element(f, b, trans_b, ldb, p, j, table);
    for (size_t i = 0; i < m; ++i) {
      double s = 0.0, g = 0.0;
      for (size_t p = 0; p < k; ++p) {
        const double x = element(f, a, trans_a, lda, i, p, table) * bcol[p];
        s += x;
        g += fabs(x);
      }
      out[i * n + j] = s;
      if (mag) mag[i * n + j] = g;
    }
  }
  free(bcol);
  free(table);
}

/* int8 x int8 -> int32, exact: products |x| <= 127 * 128 and k <= 2^17 keep every partial sum inside int32. A is
 * m x k (trans_a: stored k x m), B is k x n (trans_b: stored n x k). */
void oracle_gemm_i8(int trans_a, int trans_b, size_t m, size_t n, size_t k, const int8_t* a, size_t lda,
                    const int8_t* b, size_t ldb, int32_t* out) {
  for (size_t i = 0; i < m; ++i)
    for (size_t j = 0; j < n; ++j) {
      int64_t s = 0;
      for (size_t p = 0; p < k; ++p) {
        const int64_t x = trans_a ? a[p * lda + i] : a[i * lda + p];
        const int64_t y = trans_b ? b[j * ldb + p] : b[p * ldb + j];
        s += x * y;
      }
      out[i * n + j] = (int32_t)s;
    }
}

/* The W8A8 dequant epilogue: bf16((f32(acc) * sa[i]) * sb[j]), each multiply an f32 rounding (no FMA), then
 * narrow<bf16>. Null scales are 1. */
void oracle_dequant(size_t m, size_t n, const int32_t* acc, const float* sa, const float* sb, uint16_t* out) {
  for (size_t i = 0; i < m; ++i)
    for (size_t j = 0; j < n; ++j) {
      float v = (float)acc[i * n + j];
      if (sa) v = v * sa[i];
      if (sb) v = v * sb[j];
      int trapped;
      out[i * n + j] = (uint16_t)oracle_narrow(BF16, (double)v, &trapped);
    }
}

/* GELU, erf form, in fp64: the closed form the device's f32 epilogue is held to. */
double oracle_gelu(double x) { return 0.5 * x * (1.0 + erf(x * 0.70710678118654752440)); }

/* Narrow a whole f32 array to a storage format (bf16 output rounding of the device epilogue). */
void oracle_narrow_f32_array(int f, size_t count, const float* in, uint16_t* out) {
  for (size_t i = 0; i < count; ++i) {
    int trapped;
    out[i] = (uint16_t)oracle_narrow(f, (double)in[i], &trapped);
  }
}

/* The build's own row-parallel variant of the reference loop, for the CPU baseline only (not the reference): rows
 * [r0, r1) of the same loop, so threads that take disjoint row ranges give the reference's bits. */
void oracle_mma_rows(int f, size_t r0, size_t r1, size_t n, size_t k, float* c, const void* a, const void* b,
                     const float* table) {
  float* row = malloc((n ? n : 1) * sizeof(float));
  for (size_t i = r0; i < r1; ++i)
    for (size_t p = 0; p < k; ++p) {
      const float x = table ? table[pattern_at(f, a, i * k + p)] : ((const float*)a)[i * k + p];
      if (table)
        for (size_t j = 0; j < n; ++j) row[j] = table[pattern_at(f, b, p * n + j)];
      const float* r = table ? row : (const float*)b + p * n;
      for (size_t j = 0; j < n; ++j) c[i * n + j] = c[i * n + j] + x * r[j];
    }
  free(row);
}

/* A decode table the row-parallel variant shares between threads; free with oracle_free. */
/* oracle_quantize_rows: q[i][j] = quantize[T](x[i][j], s_i) with the reference's element function above. s_i is
 * scale[i] (mode 1), scale[0] (mode 2), or (mode 0) computed and written to scale[i]: the largest |x[i][j]| of the
 * row's non-NaN elements divided in f32 by T's largest finite value (127, 448, 57344), or 1 for a row without a
 * nonzero one. Where the reference would trap the row (a scale not positive and finite) is zeros and bit 1 of
 * *status is set; a NaN into int8 gives 0 and sets bit 2. x_type is F32, F16 or BF16; q_type 5 (int8), F8E4M3 or
 * F8E5M2. */
void oracle_quantize_rows(int x_type, int q_type, int mode, size_t m, size_t k, const void* x, size_t ldx, uint8_t* q,
                          size_t ldq, float* scale, int* status) {
  const float range = q_type == 5 ? 127.0f : q_type == F8E4M3 ? 448.0f : 57344.0f;
  float* row = malloc((k ? k : 1) * sizeof(float));
  for (size_t i = 0; i < m; ++i) {
    for (size_t j = 0; j < k; ++j)
      row[j] = x_type == F32 ? ((const float*)x)[i * ldx + j]
                             : (float)oracle_decode(x_type, ((const uint16_t*)x)[i * ldx + j]);
    float s;
    if (mode == 0) {
      float top = 0.0f;
      for (size_t j = 0; j < k; ++j) {
        const float a = fabsf(row[j]);
        if (a == a && a > top) top = a;
      }
      s = top == 0.0f ? 1.0f : top / range;
      scale[i] = s;
    } else {
      s = scale[mode == 1 ? i : 0];
    }
    if (!(s > 0.0f) || !(s <= 3.4028234663852886e38f)) {
      *status |= 1;
      memset(q + i * ldq, 0, k);
      continue;
    }
    for (size_t j = 0; j < k; ++j) {
      int trapped = 0;
      if (q_type == 5) {
        const int64_t v = oracle_quantize_int(row[j], s, -128, 127, &trapped);
        q[i * ldq + j] = (uint8_t)(trapped ? 0 : (int8_t)v);
      } else {
        q[i * ldq + j] = (uint8_t)oracle_quantize_float(q_type, row[j], s, &trapped);
      }
      if (trapped) *status |= 2;
    }
  }
  free(row);
}

float* oracle_table(int f) { return f == F32 ? NULL : decode_table(f); }
void oracle_free(void* p) { free(p); }
