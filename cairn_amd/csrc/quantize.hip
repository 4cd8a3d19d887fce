// Device quantize: quantize[T](x, scale) (src/cairn/runtime/cairn_float.hpp:116-146) over every element of an m x k
// row-major matrix, into int8 (the W8A8 operand) or an 8-bit float, with one scale per row (the caller's, one for
// the whole matrix, or the row's largest magnitude over T's range, computed here in the same pass).
//
// The kernel is bound by HBM: it reads x once and writes q once (3 bytes an element for bf16 into int8). A workgroup
// quantizes one row. Each thread holds 8-element chunks of the row in registers, so with a computed scale the row is
// read once: the largest magnitude is reduced across the workgroup, the scale follows, and the held chunks are
// quantized. Rows longer than the chunks held (256 threads x 8 x HOLD elements) are read twice, the second time
// from cache. The element arithmetic is quantize.hpp's: an f32 shortcut where it decides, the reference's double
// steps where it does not, so every output equals the reference's.
#include <hip/hip_runtime.h>
#include "../../include/cairn_gemm.h"
#include "quantize.hpp"

namespace cairn::quant {

constexpr int THREADS = 256, CHUNK = 8, HOLD = 4;
constexpr std::int64_t SPAN = std::int64_t(THREADS) * CHUNK * HOLD;  // the elements a pass holds

struct Params {
  const void* x;
  void* q;
  float* scale;
  std::int32_t* status;
  std::int64_t k, ldx, ldq;
  int mode;
};

typedef std::uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef std::uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Chunk j of this thread's part of the span at `base`: elements [col, col + 8) of the row, zeros past k.
template<int XT, bool VEC>
__device__ __forceinline__ void load_chunk(const char* row, std::int64_t col, std::int64_t k, float (&v)[CHUNK]) {
  constexpr int XS = XT == CAIRN_TYPE_F32 ? 4 : 2;
  if constexpr(VEC) {  // k, the leading dimension and the base are multiples of 8 elements: whole chunks
    const bool in = col < k;
    if constexpr(XT == CAIRN_TYPE_F32) {
      u32x4 w0 = {0, 0, 0, 0}, w1 = {0, 0, 0, 0};
      if(in) {
        w0 = *reinterpret_cast<const u32x4*>(row + col * 4);
        w1 = *reinterpret_cast<const u32x4*>(row + col * 4 + 16);
      }
      // Each element through a scalar: this compiler's __builtin_bit_cast of a vector element w[e] reads element 0.
#pragma unroll
      for(int e = 0; e < 4; ++e) {
        const std::uint32_t lo = w0[e], hi = w1[e];
        v[e] = __builtin_bit_cast(float, lo);
        v[4 + e] = __builtin_bit_cast(float, hi);
      }
    } else {
      u32x4 w = {0, 0, 0, 0};
      if(in) w = *reinterpret_cast<const u32x4*>(row + col * 2);
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
    (void)XS;
  }
}

template<bool VEC>
__device__ __forceinline__ void store_chunk(char* row, std::int64_t col, std::int64_t k, const std::uint32_t (&b)[CHUNK]) {
  if(col >= k) return;
  if constexpr(VEC) {
    u32x2 w;
    w[0] = b[0] | (b[1] << 8) | (b[2] << 16) | (b[3] << 24);
    w[1] = b[4] | (b[5] << 8) | (b[6] << 16) | (b[7] << 24);
    *reinterpret_cast<u32x2*>(row + col) = w;
  } else {
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

template<int QT>
__device__ __forceinline__ std::uint32_t exact_pattern(float x, float s, bool& trapped) {
  if constexpr(QT == CAIRN_TYPE_I8) return std::uint32_t(exact_i8(x, s, trapped)) & 0xffu;
  else if constexpr(QT == CAIRN_TYPE_F8E4M3) return exact_f8<cr::f8e4m3>(x, s);
  else return exact_f8<cr::f8e5m2>(x, s);
}

template<int XT, int QT, bool VEC>
__global__ void __launch_bounds__(THREADS) quantize_rows(Params p) {
  __shared__ std::uint32_t peak[THREADS / 64];
  const int t = threadIdx.x;
  const std::int64_t row = blockIdx.x;
  constexpr int XS = XT == CAIRN_TYPE_F32 ? 4 : 2;
  const char* xr = static_cast<const char*>(p.x) + row * p.ldx * XS;
  char* qr = static_cast<char*>(p.q) + row * p.ldq;
  auto col_of = [&](std::int64_t base, int j) { return base + (std::int64_t(j) * THREADS + t) * CHUNK; };
  float v[HOLD][CHUNK];
  auto load_span = [&](std::int64_t base) {
#pragma unroll
    for(int j = 0; j < HOLD; ++j) load_chunk<XT, VEC>(xr, col_of(base, j), p.k, v[j]);
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
    if((t & 63) == 0) peak[t >> 6] = top;
    __syncthreads();
    top = most(most(peak[0], peak[1]), most(peak[2], peak[3]));
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
      for(int j = 0; j < HOLD; ++j) store_chunk<VEC>(qr, col_of(base, j), p.k, zero);
    return;
  }
  const bool fast = fast_ok(s);  // uniform
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
          if(exact[e] || !fast) b[e] = exact_pattern<QT>(v[j][e], s, trapped);
      }
      store_chunk<VEC>(qr, col_of(base, j), p.k, b);
    }
  }
  if(trapped && p.status) atomicOr(p.status, CAIRN_QUANT_NAN);
}

}  // namespace cairn::quant

namespace {

template<int XT, int QT>
hipError_t launch(const cairn::quant::Params& p, bool vec, unsigned rows, hipStream_t s) {
  using namespace cairn::quant;
  if(vec) hipLaunchKernelGGL((quantize_rows<XT, QT, true>), dim3(rows), dim3(THREADS), 0, s, p);
  else hipLaunchKernelGGL((quantize_rows<XT, QT, false>), dim3(rows), dim3(THREADS), 0, s, p);
  return hipGetLastError();
}

template<int XT>
hipError_t launch_x(int qt, const cairn::quant::Params& p, bool vec, unsigned rows, hipStream_t s) {
  if(qt == CAIRN_TYPE_I8) return launch<XT, CAIRN_TYPE_I8>(p, vec, rows, s);
  if(qt == CAIRN_TYPE_F8E4M3) return launch<XT, CAIRN_TYPE_F8E4M3>(p, vec, rows, s);
  return launch<XT, CAIRN_TYPE_F8E5M2>(p, vec, rows, s);
}

}  // namespace

extern "C" int cairn_quantize_run(const cairn_quantize_desc* d, void* stream) {
  if(!d || d->version != CAIRN_QUANTIZE_DESC_VERSION) return CAIRN_E_ARG;
  const int xt = d->x_type, qt = d->q_type;
  if(xt != CAIRN_TYPE_F32 && xt != CAIRN_TYPE_F16 && xt != CAIRN_TYPE_BF16) return CAIRN_E_TYPE;
  if(qt != CAIRN_TYPE_I8 && qt != CAIRN_TYPE_F8E4M3 && qt != CAIRN_TYPE_F8E5M2) return CAIRN_E_TYPE;
  if(d->mode != CAIRN_SCALE_ROW_ABSMAX && d->mode != CAIRN_SCALE_ROW && d->mode != CAIRN_SCALE_TENSOR) return CAIRN_E_ARG;
  if(d->m == 0) return CAIRN_OK;
  const std::uint64_t ldx = d->ldx ? d->ldx : d->k, ldq = d->ldq ? d->ldq : d->k;
  if(d->m > 0x7fffffffu || d->k > (1ull << 40) || ldx < d->k || ldq < d->k || ldx > (1ull << 40) || ldq > (1ull << 40))
    return CAIRN_E_SHAPE;
  if(!d->scale || (d->k && (!d->x || !d->q))) return CAIRN_E_ARG;
  const int xs = xt == CAIRN_TYPE_F32 ? 4 : 2;
  const bool vec = d->k % 8 == 0 && ldx % 8 == 0 && ldq % 8 == 0 && reinterpret_cast<std::uintptr_t>(d->x) % 16 == 0 &&
                   reinterpret_cast<std::uintptr_t>(d->q) % 8 == 0;
  (void)xs;
  const cairn::quant::Params p{d->x, d->q, d->scale, d->status, std::int64_t(d->k), std::int64_t(ldx), std::int64_t(ldq),
                               d->mode};
  const auto s = static_cast<hipStream_t>(stream);
  const unsigned rows = unsigned(d->m);
  hipError_t e;
  if(xt == CAIRN_TYPE_F32) e = launch_x<CAIRN_TYPE_F32>(qt, p, vec, rows, s);
  else if(xt == CAIRN_TYPE_F16) e = launch_x<CAIRN_TYPE_F16>(qt, p, vec, rows, s);
  else e = launch_x<CAIRN_TYPE_BF16>(qt, p, vec, rows, s);
  return e == hipSuccess ? CAIRN_OK : CAIRN_E_HIP;
}
