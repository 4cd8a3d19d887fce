// Device quantize: quantize[T](x, scale) (src/cairn/runtime/cairn_float.hpp:116-146) over every element of an m x k
// row-major matrix, into int8 (the W8A8 operand) or an 8-bit float, with one scale per row (the caller's, one for
// the whole matrix, or the row's largest magnitude over T's range, computed here in the same pass).
//
// The kernel is bound by HBM: it reads x once and writes q once (3 bytes an element for bf16 into int8). A wave
// quantizes a row of up to 4096 elements (four rows a workgroup), a workgroup a longer one. Each lane holds 8-element
// chunks of the row in registers, so with a computed scale the row is read once: the largest magnitude is reduced
// across the wave (and the workgroup), the scale follows, and the held chunks are quantized. Rows longer than the
// chunks held (8192 elements for a workgroup) are read twice, the second time from cache. The element arithmetic is
// quantize.hpp's, so every output equals the reference's: for int8 an f32 shortcut where it decides and the
// reference's double steps where it does not; for the 8-bit floats the hardware's conversion, with elements near a
// midpoint of the grid settled from the neighbouring codes (convert_f8), and the integer steps for saturation and
// special values.
#include <hip/hip_runtime.h>
#include <cstdio>
#include "../../include/cairn_gemm.h"
#include "quantize.hpp"

namespace cairn::quant {

constexpr int THREADS = 256, CHUNK = 8;
// A row of at most SHORT elements is one wave's (4 rows a workgroup, no barrier); a longer one the workgroup's.
constexpr std::int64_t SHORT = 64 * CHUNK * 8;

struct Params {
  const void* x;
  void* q;
  float* scale;
  std::int32_t* status;
  std::int64_t m, k, ldx, ldq;
  int mode;
};

typedef std::uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef std::uint32_t u32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ __amdgpu_buffer_rsrc_t span_of(const void* base, std::int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, int(bytes), 0x00020000);
}

// Elements [col, col + 8) of a row. VEC: k, the leading dimension and the row's base are multiples of 8 elements, so
// a chunk is in the row or past it whole, and the row's buffer range (k elements) makes the hardware return zeros
// past k, with no branch. Otherwise element by element, zeros past k.
template<int XT, bool VEC>
__device__ __forceinline__ void load_chunk(const char* row, __amdgpu_buffer_rsrc_t rs, std::int64_t col, std::int64_t k,
                                           float (&v)[CHUNK]) {
  if constexpr(VEC) {
    if constexpr(XT == CAIRN_TYPE_F32) {
      const u32x4 w0 = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, int(col * 4), 0, 0));
      const u32x4 w1 = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, int(col * 4) + 16, 0, 0));
      // Each element through a scalar: this compiler's __builtin_bit_cast of a vector element w[e] reads element 0.
#pragma unroll
      for(int e = 0; e < 4; ++e) {
        const std::uint32_t lo = w0[e], hi = w1[e];
        v[e] = __builtin_bit_cast(float, lo);
        v[4 + e] = __builtin_bit_cast(float, hi);
      }
    } else {
      const u32x4 w = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, int(col * 2), 0, 0));
#pragma unroll
      for(int e = 0; e < 4; ++e) {
        const std::uint32_t lo = w[e] & 0xffffu, hi = w[e] >> 16;
        if constexpr(XT == CAIRN_TYPE_BF16) {
          v[2 * e] = __builtin_bit_cast(float, lo << 16);
          v[2 * e + 1] = __builtin_bit_cast(float, hi << 16);
        } else {
          v[2 * e] = float(__builtin_bit_cast(_Float16, std::uint16_t(lo)));
          v[2 * e + 1] = float(__builtin_bit_cast(_Float16, std::uint16_t(hi)));
        }
      }
    }
  } else {
#pragma unroll
    for(int e = 0; e < CHUNK; ++e) {
      const std::int64_t c = col + e;
      if(c >= k) {
        v[e] = 0.0f;
        continue;
      }
      if constexpr(XT == CAIRN_TYPE_F32) v[e] = reinterpret_cast<const float*>(row)[c];
      else {
        const std::uint16_t h = reinterpret_cast<const std::uint16_t*>(row)[c];
        v[e] = XT == CAIRN_TYPE_BF16 ? __builtin_bit_cast(float, std::uint32_t(h) << 16)
                                     : float(__builtin_bit_cast(_Float16, h));
      }
    }
  }
}

// The chunk's 8 patterns; VEC: one 8-byte store the row's buffer range drops past k.
template<bool VEC>
__device__ __forceinline__ void store_chunk(char* row, __amdgpu_buffer_rsrc_t rs, std::int64_t col, std::int64_t k,
                                            const std::uint32_t (&b)[CHUNK]) {
  if constexpr(VEC) {
    u32x2 w;
    w[0] = b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24);
    w[1] = b[4] | (b[5] << 8) | (b[6] << 16) | (b[7] << 24);
    __builtin_amdgcn_raw_buffer_store_b64(w, rs, int(col), 0, 0);
  } else {
    if(col >= k) return;
#pragma unroll
    for(int e = 0; e < CHUNK; ++e)
      if(col + e < k) reinterpret_cast<std::uint8_t*>(row)[col + e] = std::uint8_t(b[e]);
  }
}

// The magnitude bits of v, NaN counted as 0: for non-negative floats the bit patterns order as the values do.
__device__ __forceinline__ std::uint32_t magnitude(float v) {
  const std::uint32_t m = __builtin_bit_cast(std::uint32_t, v) & 0x7fffffffu;
  return m > 0x7f800000u ? 0u : m;
}

__device__ __forceinline__ std::uint32_t most(std::uint32_t a, std::uint32_t b) { return a > b ? a : b; }

// Element e of a chunk, into its pattern (int8 as its two's-complement byte). `exact` marks what the shortcut left.
template<int QT>
__device__ __forceinline__ std::uint32_t shortcut(float x, float r, bool& exact) {
  if constexpr(QT == CAIRN_TYPE_I8) {
    int v;
    exact = !try_i8(x * r, v);
    return std::uint32_t(v) & 0xffu;
  } else {
    using T = std::conditional_t<QT == CAIRN_TYPE_F8E4M3, cr::f8e4m3, cr::f8e5m2>;
    std::uint32_t out;
    exact = !try_f8<T>(x, x * r, out);
    return out;
  }
}

// What the shortcut left: with the scale in the shortcut's range (`fast`) and x not a NaN, the fma decision on y;
// otherwise the reference's double steps.
template<int QT>
__device__ __forceinline__ std::uint32_t exact_pattern(float x, float s, float r, bool fast, bool& trapped) {
  using T = std::conditional_t<QT == CAIRN_TYPE_F8E4M3, cr::f8e4m3, cr::f8e5m2>;
  if constexpr(QT == CAIRN_TYPE_I8) {
    if(fast && x == x) return std::uint32_t(near_i8(x, s, x * r)) & 0xffu;
    return std::uint32_t(exact_i8(x, s, trapped)) & 0xffu;
  } else {
    if(fast && x == x) return near_f8<T>(x, s, x * r);
    return exact_f8<T>(x, s);
  }
}

// Whether the shortcut (and the fma decision) are sound for this scale: a property of the row, so uniform.
template<int QT> __device__ __forceinline__ bool fast_for(float s) {
  return QT == CAIRN_TYPE_I8 ? fast_ok(s) : fast_ok_f8(s);
}

// ROWS rows a workgroup: 4 (a wave a row) or 1 (the workgroup a row); each lane holds HOLD chunks a pass (the generic
// kernel: 8 or 4, so rows up to SHORT or 8192 elements are read once; the fast kernel's rare rows: 1, to keep its
// registers for the common case). The row of thread t (t < 256 / ROWS), element by element through the shortcut and
// the exact path: every case, NaN and scales outside the shortcut's range included.
template<int XT, int QT, bool VEC, int ROWS, int HOLD>
__device__ void generic_row(const Params& p, std::int64_t row, int t, std::uint32_t* peak) {
  constexpr int RT = THREADS / ROWS;
  constexpr std::int64_t SPAN = std::int64_t(RT) * CHUNK * HOLD;  // the elements a pass holds
  constexpr int XS = XT == CAIRN_TYPE_F32 ? 4 : 2;
  const char* xr = static_cast<const char*>(p.x) + row * p.ldx * XS;
  char* qr = static_cast<char*>(p.q) + row * p.ldq;
  const __amdgpu_buffer_rsrc_t xs = span_of(xr, p.k * XS), qs = span_of(qr, p.k);
  auto col_of = [&](std::int64_t base, int j) { return base + (std::int64_t(j) * RT + t) * CHUNK; };
  float v[HOLD][CHUNK];
  auto load_span = [&](std::int64_t base) {
#pragma unroll
    for(int j = 0; j < HOLD; ++j) load_chunk<XT, VEC>(xr, xs, col_of(base, j), p.k, v[j]);
  };

  float s;
  if(p.mode == CAIRN_SCALE_ROW_ABSMAX) {
    std::uint32_t top = 0;
    for(std::int64_t base = 0; base < p.k; base += SPAN) {
      load_span(base);
#pragma unroll
      for(int j = 0; j < HOLD; ++j)
#pragma unroll
        for(int e = 0; e < CHUNK; ++e) top = most(top, magnitude(v[j][e]));
    }
#pragma unroll
    for(int o = 32; o >= 1; o >>= 1) top = most(top, std::uint32_t(__shfl_xor(int(top), o)));
    if constexpr(ROWS == 1) {
      if((t & 63) == 0) peak[t >> 6] = top;
      __syncthreads();
      top = most(most(peak[0], peak[1]), most(peak[2], peak[3]));
    }
    const float largest = __builtin_bit_cast(float, top);
    using T = std::conditional_t<QT == CAIRN_TYPE_F8E4M3, cr::f8e4m3, cr::f8e5m2>;
    s = largest == 0.0f ? 1.0f : largest / (QT == CAIRN_TYPE_I8 ? 127.0f : range_of<T>());
    if(t == 0) p.scale[row] = s;
  } else {
    s = p.scale[p.mode == CAIRN_SCALE_ROW ? row : 0];
    if(p.k > 0) load_span(0);
  }

  if(!scale_ok(s)) {  // the reference traps: the row is written as zeros and the status says so
    if(t == 0 && p.status) atomicOr(p.status, CAIRN_QUANT_BAD_SCALE);
    const std::uint32_t zero[CHUNK] = {};
    for(std::int64_t base = 0; base < p.k; base += SPAN)
#pragma unroll
      for(int j = 0; j < HOLD; ++j) store_chunk<VEC>(qr, qs, col_of(base, j), p.k, zero);
    return;
  }
  const bool fast = fast_for<QT>(s);  // uniform
  const float r = 1.0f / s;
  bool trapped = false;
  for(std::int64_t base = 0; base < p.k; base += SPAN) {
    if(base > 0 || (p.mode == CAIRN_SCALE_ROW_ABSMAX && p.k > SPAN)) load_span(base);  // the first span is held
#pragma unroll
    for(int j = 0; j < HOLD; ++j) {
      std::uint32_t b[CHUNK];
      bool exact[CHUNK], any = !fast;
#pragma unroll
      for(int e = 0; e < CHUNK; ++e) {
        exact[e] = false;
        b[e] = shortcut<QT>(v[j][e], r, exact[e]);
        any |= exact[e];
      }
      if(any) {  // rare: an element near a rounding boundary, a NaN, or a scale outside the shortcut's range
#pragma unroll
        for(int e = 0; e < CHUNK; ++e)
          if(exact[e] || !fast) b[e] = exact_pattern<QT>(v[j][e], s, r, fast, trapped);
      }
      store_chunk<VEC>(qr, qs, col_of(base, j), p.k, b);
    }
  }
  if(trapped && p.status) atomicOr(p.status, CAIRN_QUANT_NAN);
}

// The row of each wave (ROWS = 4) or workgroup (ROWS = 1). The row is uniform, so its buffer ranges live in scalar
// registers.
template<int ROWS>
__device__ __forceinline__ std::int64_t row_of() {
  return std::int64_t(blockIdx.x) * ROWS + __builtin_amdgcn_readfirstlane(int(threadIdx.x / (THREADS / ROWS)));
}

template<int XT, int QT, bool VEC, int ROWS>
__global__ void __launch_bounds__(THREADS) quantize_rows(Params p) {
  __shared__ std::uint32_t peak[THREADS / 64];
  const std::int64_t row = row_of<ROWS>();
  if(row >= p.m) return;  // a wave past the last row (ROWS = 4); no barrier follows in that case
  generic_row<XT, QT, VEC, ROWS, ROWS == 1 ? 4 : 8>(p, row, int(threadIdx.x % (THREADS / ROWS)), peak);
}

// ---- The fast kernel: whole chunks (VEC), rows without NaN, scales in the shortcut's range.

// A chunk of 8 elements as loaded: one 16-byte word of 16-bit patterns, or two of f32.
template<int XT> struct Raw {
  u32x4 w[XT == CAIRN_TYPE_F32 ? 2 : 1];
};

template<int XT>
__device__ __forceinline__ void load_raw(__amdgpu_buffer_rsrc_t rs, std::int64_t col, Raw<XT>& r) {
  if constexpr(XT == CAIRN_TYPE_F32) {
    r.w[0] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, int(col * 4), 0, 0));
    r.w[1] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, int(col * 4) + 16, 0, 0));
  } else {
    r.w[0] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, int(col * 2), 0, 0));
  }
}

// Element e as f32, exactly (each through a scalar: see load_chunk).
template<int XT>
__device__ __forceinline__ float element(const Raw<XT>& r, int e) {
  if constexpr(XT == CAIRN_TYPE_F32) {
    const std::uint32_t u = r.w[e >> 2][e & 3];
    return __builtin_bit_cast(float, u);
  } else {
    const std::uint32_t u = r.w[0][e >> 1];
    if constexpr(XT == CAIRN_TYPE_BF16) return __builtin_bit_cast(float, (e & 1) ? (u & 0xffff0000u) : (u << 16));
    else return float(__builtin_bit_cast(_Float16, std::uint16_t((e & 1) ? (u >> 16) : (u & 0xffffu))));
  }
}

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

// The largest magnitude pattern so far, NaN patterns included (they order above infinity): one packed 16-bit max
// for two 16-bit elements (two maxima kept in `top`'s halves), one 32-bit max an f32 element.
template<int XT>
__device__ __forceinline__ void pattern_max(const Raw<XT>& r, std::uint32_t& top) {
  if constexpr(XT == CAIRN_TYPE_F32) {
#pragma unroll
    for(int i = 0; i < 2; ++i)
#pragma unroll
      for(int e = 0; e < 4; ++e) {
        const std::uint32_t u = r.w[i][e];
        top = most(top, u & 0x7fffffffu);
      }
  } else {
    u16x2 acc = __builtin_bit_cast(u16x2, top);
#pragma unroll
    for(int e = 0; e < 4; ++e) {
      const std::uint32_t u = r.w[0][e] & 0x7fff7fffu;
      acc = __builtin_elementwise_max(acc, __builtin_bit_cast(u16x2, u));
    }
    top = __builtin_bit_cast(std::uint32_t, acc);
  }
}

// The maximum over the wave's 64 lanes: within each row of 16 lanes by DPP (quad swaps, then the half-row and row
// mirrors), then across the four rows by reading one lane of each.
__device__ __forceinline__ std::uint32_t wave_max(std::uint32_t v) {
  v = most(v, std::uint32_t(__builtin_amdgcn_update_dpp(0, int(v), 0xB1, 0xF, 0xF, false)));   // quad_perm 1,0,3,2
  v = most(v, std::uint32_t(__builtin_amdgcn_update_dpp(0, int(v), 0x4E, 0xF, 0xF, false)));   // quad_perm 2,3,0,1
  v = most(v, std::uint32_t(__builtin_amdgcn_update_dpp(0, int(v), 0x141, 0xF, 0xF, false)));  // row_half_mirror
  v = most(v, std::uint32_t(__builtin_amdgcn_update_dpp(0, int(v), 0x140, 0xF, 0xF, false)));  // row_mirror
  const std::uint32_t a = std::uint32_t(__builtin_amdgcn_readlane(int(v), 0));
  const std::uint32_t b = std::uint32_t(__builtin_amdgcn_readlane(int(v), 16));
  const std::uint32_t c = std::uint32_t(__builtin_amdgcn_readlane(int(v), 32));
  const std::uint32_t d = std::uint32_t(__builtin_amdgcn_readlane(int(v), 48));
  return most(most(a, b), most(c, d));
}

// int8 patterns of a chunk packed four to a word (v_perm picks each value's low byte).
__device__ __forceinline__ u32x2 pack_i8(const int (&c)[CHUNK]) {
  u32x2 o;
#pragma unroll
  for(int h = 0; h < 2; ++h) {
    const std::uint32_t lo = __builtin_amdgcn_perm(std::uint32_t(c[4 * h + 1]), std::uint32_t(c[4 * h]), 0x0c0c0400u);
    const std::uint32_t hi = __builtin_amdgcn_perm(std::uint32_t(c[4 * h + 3]), std::uint32_t(c[4 * h + 2]), 0x04000c0cu);
    o[h] = lo | hi;
  }
  return o;
}

// A chunk into the 8-bit float QT through the hardware's conversions, four codes a word (convert_f8 in quantize.hpp
// states when its answer is the reference's).
template<int QT> __device__ __forceinline__ bool hw_f8(const float (&x)[CHUNK], const float (&y)[CHUNK], float s,
                                                       u32x2& o) {
  using T = std::conditional_t<QT == CAIRN_TYPE_F8E4M3, cr::f8e4m3, cr::f8e5m2>;
  std::uint32_t w[2];
  const bool ok = convert_f8<T>(
      x, y, s, w,
      [](float a, float b, float c, float d) {
        if constexpr(QT == CAIRN_TYPE_F8E4M3)
          return std::uint32_t(
              __builtin_amdgcn_cvt_pk_fp8_f32(c, d, __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false), true));
        else
          return std::uint32_t(
              __builtin_amdgcn_cvt_pk_bf8_f32(c, d, __builtin_amdgcn_cvt_pk_bf8_f32(a, b, 0, false), true));
      },
      [](std::uint32_t code) {
        if constexpr(QT == CAIRN_TYPE_F8E4M3) return __builtin_amdgcn_cvt_f32_fp8(int(code), 0);
        else return __builtin_amdgcn_cvt_f32_bf8(int(code), 0);
      });
  o[0] = w[0];
  o[1] = w[1];
  return ok;
}

template<int XT, int QT, int ROWS>
__global__ void __launch_bounds__(THREADS) quantize_fast(Params p) {
  constexpr int RT = THREADS / ROWS, HOLD = ROWS == 1 ? 4 : 8;
  constexpr std::int64_t SPAN = std::int64_t(RT) * CHUNK * HOLD;
  constexpr int XS = XT == CAIRN_TYPE_F32 ? 4 : 2;
  constexpr std::uint32_t INF = XT == CAIRN_TYPE_F32 ? 0x7f800000u : XT == CAIRN_TYPE_BF16 ? 0x7f80u : 0x7c00u;
  __shared__ std::uint32_t peak[THREADS / 64];
  const std::int64_t row = row_of<ROWS>();
  if(row >= p.m) return;  // a wave past the last row (ROWS = 4); no barrier follows in that case
  const int t = int(threadIdx.x % RT);
  const char* xr = static_cast<const char*>(p.x) + row * p.ldx * XS;
  char* qr = static_cast<char*>(p.q) + row * p.ldq;
  const __amdgpu_buffer_rsrc_t xs = span_of(xr, p.k * XS), qs = span_of(qr, p.k);
  auto col_of = [&](std::int64_t base, int j) { return base + (std::int64_t(j) * RT + t) * CHUNK; };
  Raw<XT> w[HOLD];
  auto load_span = [&](std::int64_t base) {
#pragma unroll
    for(int j = 0; j < HOLD; ++j) load_raw<XT>(xs, col_of(base, j), w[j]);
  };

  std::uint32_t top = 0;
  for(std::int64_t base = 0; base < p.k; base += SPAN) {
    load_span(base);
#pragma unroll
    for(int j = 0; j < HOLD; ++j) pattern_max<XT>(w[j], top);
  }
  if constexpr(XT != CAIRN_TYPE_F32) top = most(top & 0xffffu, top >> 16);
  top = wave_max(top);
  if constexpr(ROWS == 1) {
    if((t & 63) == 0) peak[t >> 6] = top;
    __syncthreads();
    top = most(most(peak[0], peak[1]), most(peak[2], peak[3]));
    __syncthreads();  // every wave has read `peak` before the generic path may write it
  }
  if(top > INF) {  // a NaN in the row (uniform): the generic path leaves it out of the scale and reports it
    generic_row<XT, QT, true, ROWS, 1>(p, row, t, peak);
    return;
  }
  float s;
  if(p.mode == CAIRN_SCALE_ROW_ABSMAX) {
    float largest;
    if constexpr(XT == CAIRN_TYPE_F32) largest = __builtin_bit_cast(float, top);
    else if constexpr(XT == CAIRN_TYPE_BF16) largest = __builtin_bit_cast(float, top << 16);
    else largest = float(__builtin_bit_cast(_Float16, std::uint16_t(top)));
    using T = std::conditional_t<QT == CAIRN_TYPE_F8E4M3, cr::f8e4m3, cr::f8e5m2>;
    s = largest == 0.0f ? 1.0f : largest / (QT == CAIRN_TYPE_I8 ? 127.0f : range_of<T>());
    if(t == 0) p.scale[row] = s;
  } else {
    s = p.scale[p.mode == CAIRN_SCALE_ROW ? row : 0];
  }
  if(!scale_ok(s)) {  // the reference traps: the row is written as zeros and the status says so
    if(t == 0 && p.status) atomicOr(p.status, CAIRN_QUANT_BAD_SCALE);
    const u32x2 zero = {0u, 0u};
    for(std::int64_t base = 0; base < p.k; base += SPAN)
#pragma unroll
      for(int j = 0; j < HOLD; ++j) __builtin_amdgcn_raw_buffer_store_b64(zero, qs, int(col_of(base, j)), 0, 0);
    return;
  }
  if(!fast_for<QT>(s)) {  // uniform: every element by the exact path
    generic_row<XT, QT, true, ROWS, 1>(p, row, t, peak);
    return;
  }
  const float r = 1.0f / s;
  for(std::int64_t base = 0; base < p.k; base += SPAN) {
    if(p.k > SPAN) load_span(base);  // otherwise the one span is still held
#pragma unroll
    for(int j = 0; j < HOLD; ++j) {
      u32x2 o;
      if constexpr(QT == CAIRN_TYPE_I8) {
        int c[CHUNK];
        float dev = 0.0f;
#pragma unroll
        for(int e = 0; e < CHUNK; ++e) {
          float d;
          c[e] = round_i8(element<XT>(w[j], e) * r, d);
          dev = __builtin_fmaxf(dev, d);
        }
        if(dev > MARGIN_I8) {  // an element near a tie: the fma decides it
#pragma unroll
          for(int e = 0; e < CHUNK; ++e) {
            const float x = element<XT>(w[j], e);
            float d;
            round_i8(x * r, d);
            if(d > MARGIN_I8) c[e] = near_i8(x, s, x * r);
          }
        }
        o = pack_i8(c);
      } else {
        using T = std::conditional_t<QT == CAIRN_TYPE_F8E4M3, cr::f8e4m3, cr::f8e5m2>;
        float x[CHUNK], y[CHUNK];
#pragma unroll
        for(int e = 0; e < CHUNK; ++e) {
          x[e] = element<XT>(w[j], e);
          y[e] = x[e] * r;
        }
        if(!hw_f8<QT>(x, y, s, o)) {  // saturation, infinity, NaN: rare; the integer steps decide
          std::uint32_t b[CHUNK];
#pragma unroll
          for(int e = 0; e < CHUNK; ++e)
            if(!try_f8<T>(x[e], y[e], b[e])) b[e] = near_f8<T>(x[e], s, y[e]);
          o[0] = b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24);
          o[1] = b[4] | (b[5] << 8) | (b[6] << 16) | (b[7] << 24);
        }
      }
      __builtin_amdgcn_raw_buffer_store_b64(o, qs, int(col_of(base, j)), 0, 0);
    }
  }
}

}  // namespace cairn::quant

namespace {

template<int XT, int QT>
hipError_t launch(const cairn::quant::Params& p, bool vec, unsigned rows, hipStream_t s) {
  using namespace cairn::quant;
  const dim3 block(THREADS), by_wave((rows + 3) / 4), by_group(rows);
  if(p.k <= SHORT) {
    if(vec) hipLaunchKernelGGL((quantize_fast<XT, QT, 4>), by_wave, block, 0, s, p);
    else hipLaunchKernelGGL((quantize_rows<XT, QT, false, 4>), by_wave, block, 0, s, p);
  } else {
    if(vec) hipLaunchKernelGGL((quantize_fast<XT, QT, 1>), by_group, block, 0, s, p);
    else hipLaunchKernelGGL((quantize_rows<XT, QT, false, 1>), by_group, block, 0, s, p);
  }
  return hipGetLastError();
}

template<int XT>
hipError_t launch_x(int qt, const cairn::quant::Params& p, bool vec, unsigned rows, hipStream_t s) {
  if(qt == CAIRN_TYPE_I8) return launch<XT, CAIRN_TYPE_I8>(p, vec, rows, s);
  if(qt == CAIRN_TYPE_F8E4M3) return launch<XT, CAIRN_TYPE_F8E4M3>(p, vec, rows, s);
  return launch<XT, CAIRN_TYPE_F8E5M2>(p, vec, rows, s);
}

// The checks cairn_quantize_run makes before it launches: CAIRN_OK with `vec` (whole aligned 8-element chunks, the
// fast kernel's form) set, or the refusal.
int checked(const cairn_quantize_desc* d, bool& vec) {
  if(!d || d->version != CAIRN_QUANTIZE_DESC_VERSION) return CAIRN_E_ARG;
  const int xt = d->x_type, qt = d->q_type;
  if(xt != CAIRN_TYPE_F32 && xt != CAIRN_TYPE_F16 && xt != CAIRN_TYPE_BF16) return CAIRN_E_TYPE;
  if(qt != CAIRN_TYPE_I8 && qt != CAIRN_TYPE_F8E4M3 && qt != CAIRN_TYPE_F8E5M2) return CAIRN_E_TYPE;
  if(d->mode != CAIRN_SCALE_ROW_ABSMAX && d->mode != CAIRN_SCALE_ROW && d->mode != CAIRN_SCALE_TENSOR) return CAIRN_E_ARG;
  if(d->m == 0) return CAIRN_OK;  // nothing to launch
  const std::uint64_t ldx = d->ldx ? d->ldx : d->k, ldq = d->ldq ? d->ldq : d->k;
  // A row is addressed through a buffer range of k elements: k * 4 bytes must fit its 31-bit offsets.
  if(d->m > 0x7fffffffu || d->k > (1ull << 28) || ldx < d->k || ldq < d->k || ldx > (1ull << 40) || ldq > (1ull << 40))
    return CAIRN_E_SHAPE;
  if(!d->scale || (d->k && (!d->x || !d->q))) return CAIRN_E_ARG;
  vec = d->k % 8 == 0 && ldx % 8 == 0 && ldq % 8 == 0 && reinterpret_cast<std::uintptr_t>(d->x) % 16 == 0 &&
        reinterpret_cast<std::uintptr_t>(d->q) % 8 == 0;
  return CAIRN_OK;
}

const char* type_name(int t) {
  switch(t) {
    case CAIRN_TYPE_F32: return "f32";
    case CAIRN_TYPE_F16: return "f16";
    case CAIRN_TYPE_BF16: return "bf16";
    case CAIRN_TYPE_I8: return "i8";
    case CAIRN_TYPE_F8E4M3: return "f8e4m3";
    default: return "f8e5m2";
  }
}

}  // namespace

extern "C" int cairn_quantize_run(const cairn_quantize_desc* d, void* stream) {
  bool vec = false;
  if(const int s = checked(d, vec); s != CAIRN_OK) return s;
  if(d->m == 0) return CAIRN_OK;
  const std::uint64_t ldx = d->ldx ? d->ldx : d->k, ldq = d->ldq ? d->ldq : d->k;
  const cairn::quant::Params p{d->x,          d->q,          d->scale,           d->status,          std::int64_t(d->m),
                               std::int64_t(d->k), std::int64_t(ldx), std::int64_t(ldq), d->mode};
  const auto s = static_cast<hipStream_t>(stream);
  const unsigned rows = unsigned(d->m);
  hipError_t e;
  if(d->x_type == CAIRN_TYPE_F32) e = launch_x<CAIRN_TYPE_F32>(d->q_type, p, vec, rows, s);
  else if(d->x_type == CAIRN_TYPE_F16) e = launch_x<CAIRN_TYPE_F16>(d->q_type, p, vec, rows, s);
  else e = launch_x<CAIRN_TYPE_BF16>(d->q_type, p, vec, rows, s);
  return e == hipSuccess ? CAIRN_OK : CAIRN_E_HIP;
}

extern "C" const char* cairn_quantize_kernel(const cairn_quantize_desc* d) {
  bool vec = false;
  if(checked(d, vec) != CAIRN_OK || d->m == 0) return nullptr;
  // One name a form: the kernel family, the element types, and the rows a workgroup (4 short rows, 1 long one).
  static char names[2][3][3][2][40];
  static const bool made = [] {
    const int xs[3] = {CAIRN_TYPE_F32, CAIRN_TYPE_F16, CAIRN_TYPE_BF16};
    const int qs[3] = {CAIRN_TYPE_I8, CAIRN_TYPE_F8E4M3, CAIRN_TYPE_F8E5M2};
    for(int v = 0; v < 2; ++v)
      for(int x = 0; x < 3; ++x)
        for(int q = 0; q < 3; ++q)
          for(int r = 0; r < 2; ++r)
            std::snprintf(names[v][x][q][r], sizeof names[v][x][q][r], "%s<%s, %s, %d>",
                          v ? "quantize_fast" : "quantize_rows", type_name(xs[x]), type_name(qs[q]), r ? 1 : 4);
    return true;
  }();
  (void)made;
  const int x = d->x_type == CAIRN_TYPE_F32 ? 0 : d->x_type == CAIRN_TYPE_F16 ? 1 : 2;
  const int q = d->q_type == CAIRN_TYPE_I8 ? 0 : d->q_type == CAIRN_TYPE_F8E4M3 ? 1 : 2;
  return names[vec][x][q][std::int64_t(d->k) > cairn::quant::SHORT];
}
