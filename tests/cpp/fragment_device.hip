// The MFMA fragments (include/cairn/cairn_fragment.hpp) on the device, in kernels shaped as CAIRN emits fragment code:
// each operation through the emitted spellings (filled, loaded, multiplied, stored, get, set) with layout lambdas.
// Built by __graft_entry__.build() into tests/cpp/libfragment_device.so; tests/test_gpu_fragment.py calls it.
//
// - frag_wave_*: one wave, C += A * B over `steps` k-steps of one shape, A, B and C through layouts given as
//   (pitch, by columns, swizzle), read from global memory or first copied into LDS tiles;
// - frag_share_*: the same product, then every lane writes its values v through get, and set's effect through a
//   store, so the host can check which element each (lane, v) is;
// - frag_tile_gemm: a whole GEMM in the shape of the reference's examples/tensor/tile64.cairn: 64 x 64 output tiles,
//   a workgroup of four waves, each a 32 x 32 accumulator, k in steps of 16 through an LDS stage.
#include <hip/hip_runtime.h>
#include <cstdint>
#include "cairn_fragment.hpp"
#include "cairn_layout.hpp"

using namespace cr::frag;

namespace {

struct Tile {
  int pitch, by_columns, swizzle;  // element (r, c) at r * pitch + c (or c * pitch + r), then Swizzle<s, 3, 3>
  __device__ std::size_t operator()(std::size_t r, std::size_t c) const {
    const std::size_t o = by_columns ? c * pitch + r : r * pitch + c;
    return swizzle == 1 ? cr::layout::swizzle<1, 3, 3>(o) : swizzle == 2 ? cr::layout::swizzle<2, 3, 3>(o) : o;
  }
};

constexpr int SHARED_BYTES = 32768;  // LDS for the copied tiles: A and B, each at most 16 KiB

// A's rows M and columns steps * K, B's rows steps * K and columns N; the tiles' cosizes bound every offset.
template<class T, int M, int N, int K>
__global__ void __launch_bounds__(64) wave_kernel(float* c32, std::int32_t* ci, const T* a, const T* b, Tile ta, Tile tb,
                                                  Tile tc, int steps, int a_cells, int b_cells, int via_lds) {
  using H = held_t<T>;
  __shared__ __attribute__((aligned(16))) char lds[SHARED_BYTES];
  const T* sa = a;
  const T* sb = b;
  if(via_lds) {  // copy both tiles element by element, then read the fragments from LDS
    T* la = reinterpret_cast<T*>(lds);
    T* lb = reinterpret_cast<T*>(lds + SHARED_BYTES / 2);
    for(int e = threadIdx.x; e < a_cells; e += 64) la[e] = a[e];
    for(int e = threadIdx.x; e < b_cells; e += 64) lb[e] = b[e];
    __syncthreads();
    sa = la;
    sb = lb;
  }
  H* cc;
  if constexpr(std::is_integral_v<H>) cc = ci;
  else cc = c32;
  auto at_c = [tc](std::size_t r, std::size_t col) { return tc(r, col); };
  auto acc = loaded<MfmaFragment<Role::acc, H, M, N, K>>(cc, at_c, std::size_t(tc.pitch), !tc.by_columns, false);
  for(int s = 0; s < steps; ++s) {
    auto at_a = [ta, s](std::size_t r, std::size_t col) { return ta(r, col + std::size_t(s) * K); };
    auto at_b = [tb, s](std::size_t r, std::size_t col) { return tb(r + std::size_t(s) * K, col); };
    const auto fa = loaded<MfmaFragment<Role::a, T, M, N, K>>(sa, at_a, std::size_t(ta.pitch), !ta.by_columns, via_lds);
    const auto fb = loaded<MfmaFragment<Role::b, T, M, N, K>>(sb, at_b, std::size_t(tb.pitch), !tb.by_columns, via_lds);
    acc = multiplied(acc, fa, fb);
  }
  stored(acc, cc, at_c, std::size_t(tc.pitch), !tc.by_columns, unsigned(threadIdx.x));
}

// C = A * B of one k-step (packed tiles), then lane l writes get(acc, v) to got[l * V + v], and sets each of its
// values to 1000 l + v before storing the accumulator into c.
template<class T, int M, int N, int K>
__global__ void __launch_bounds__(64) share_kernel(float* got, float* c, const T* a, const T* b) {
  using H = held_t<T>;
  constexpr int V = values<M, N>;
  auto rows_a = [](std::size_t r, std::size_t col) { return r * K + col; };
  auto rows_b = [](std::size_t r, std::size_t col) { return r * N + col; };
  auto rows_c = [](std::size_t r, std::size_t col) { return r * N + col; };
  auto acc = filled<MfmaFragment<Role::acc, H, M, N, K>>(0);
  acc = multiplied(acc, loaded<MfmaFragment<Role::a, T, M, N, K>>(a, rows_a, K, true, false),
                   loaded<MfmaFragment<Role::b, T, M, N, K>>(b, rows_b, N, true, false));
  const unsigned lane = threadIdx.x;
  for(int v = 0; v < V; ++v) got[lane * V + v] = float(get(acc, std::size_t(v), lane));
  for(int v = 0; v < V; ++v) acc = set(acc, std::size_t(v), H(1000 * int(lane) + v), lane);
  stored(acc, c, rows_c, N, true, lane);
}

// The tile64 shape: workgroup (tx, ty) of 256 threads computes the 64 x 64 tile (by, bx); wave w holds the 32 x 32
// accumulator (w / 2, w % 2) of it. Each k-step of 16 copies A's 64 x 16 and B's 16 x 64 slices into LDS (zero
// past the matrix), then every wave multiplies its fragments. c is read first and written last, inside the matrix.
template<class T>
__global__ void __launch_bounds__(256) tile_kernel(int m, int n, int k, float* c, const T* a, const T* b) {
  __shared__ __attribute__((aligned(16))) T sa[64 * 16];
  __shared__ __attribute__((aligned(16))) T sb[16 * 64];
  __shared__ float sc[64 * 68];  // rows 68 floats apart
  const int t = threadIdx.x, wave = t / 64, lane = t % 64;
  const int row0 = blockIdx.y * 64, col0 = blockIdx.x * 64;
  for(int e = t; e < 64 * 64; e += 256) {
    const int r = e / 64, q = e % 64;
    sc[r * 68 + q] = row0 + r < m && col0 + q < n ? c[std::size_t(row0 + r) * n + col0 + q] : 0.0f;
  }
  __syncthreads();
  const int wr = 32 * (wave / 2), wc = 32 * (wave % 2);
  auto at_c = [wr, wc](std::size_t r, std::size_t q) { return (wr + r) * 68 + wc + q; };
  auto acc = loaded<MfmaFragment<Role::acc, float, 32, 32, 16>>(sc, at_c, 68, true, true);
  const T zero{};
  for(int k0 = 0; k0 < k; k0 += 16) {
    for(int e = t; e < 64 * 16; e += 256) {
      const int r = e / 16, q = e % 16;
      sa[e] = row0 + r < m && k0 + q < k ? a[std::size_t(row0 + r) * k + k0 + q] : zero;
      const int p = e / 64, j = e % 64;
      sb[e] = k0 + p < k && col0 + j < n ? b[std::size_t(k0 + p) * n + col0 + j] : zero;
    }
    __syncthreads();
    auto at_a = [wr](std::size_t r, std::size_t q) { return (wr + r) * 16 + q; };
    auto at_b = [wc](std::size_t p, std::size_t j) { return p * 64 + wc + j; };
    acc = multiplied(acc, loaded<MfmaFragment<Role::a, T, 32, 32, 16>>(sa, at_a, 16, true, true),
                     loaded<MfmaFragment<Role::b, T, 32, 32, 16>>(sb, at_b, 64, true, true));
    __syncthreads();  // every wave's reads of this step before the next copy
  }
  stored(acc, sc, at_c, 68, true, unsigned(lane));
  __syncthreads();
  for(int e = t; e < 64 * 64; e += 256) {
    const int r = e / 64, q = e % 64;
    if(row0 + r < m && col0 + q < n) c[std::size_t(row0 + r) * n + col0 + q] = sc[r * 68 + q];
  }
}

template<class F> int launched(F&& launch) {
  launch();
  return hipGetLastError() == hipSuccess ? 0 : 1;
}

}  // namespace

#define WAVE_ENTRY(NAME, T, M, N, K)                                                                                  \
  extern "C" int NAME(float* c32, std::int32_t* ci, const void* a, const void* b, const int* ta, const int* tb,       \
                      const int* tc, int steps, int a_cells, int b_cells, int via_lds) {                             \
    if(a_cells * int(sizeof(T)) > SHARED_BYTES / 2 || b_cells * int(sizeof(T)) > SHARED_BYTES / 2) return 2;       \
    return launched([&] {                                                                                            \
      hipLaunchKernelGGL((wave_kernel<T, M, N, K>), dim3(1), dim3(64), 0, 0, c32, ci, static_cast<const T*>(a),    \
                         static_cast<const T*>(b), Tile{ta[0], ta[1], ta[2]}, Tile{tb[0], tb[1], tb[2]},            \
                         Tile{tc[0], tc[1], tc[2]}, steps, a_cells, b_cells, via_lds);                               \
    });                                                                                                              \
  }
WAVE_ENTRY(frag_wave_bf16_32x32x16, cr::bf16, 32, 32, 16)
WAVE_ENTRY(frag_wave_f16_32x32x16, cr::f16, 32, 32, 16)
WAVE_ENTRY(frag_wave_bf16_16x16x32, cr::bf16, 16, 16, 32)
WAVE_ENTRY(frag_wave_f16_16x16x32, cr::f16, 16, 16, 32)
WAVE_ENTRY(frag_wave_i8_32x32x32, std::int8_t, 32, 32, 32)

#define SHARE_ENTRY(NAME, T, M, N, K)                                                                                 \
  extern "C" int NAME(float* got, float* c, const void* a, const void* b) {                                          \
    return launched([&] {                                                                                            \
      hipLaunchKernelGGL((share_kernel<T, M, N, K>), dim3(1), dim3(64), 0, 0, got, c, static_cast<const T*>(a),     \
                         static_cast<const T*>(b));                                                                  \
    });                                                                                                              \
  }
SHARE_ENTRY(frag_share_bf16_32x32x16, cr::bf16, 32, 32, 16)
SHARE_ENTRY(frag_share_bf16_16x16x32, cr::bf16, 16, 16, 32)

extern "C" int frag_tile_gemm(int type, int m, int n, int k, float* c, const void* a, const void* b) {
  if(m <= 0 || n <= 0 || k < 0) return 2;
  const dim3 grid(unsigned((n + 63) / 64), unsigned((m + 63) / 64));
  return launched([&] {
    if(type == 2)
      hipLaunchKernelGGL((tile_kernel<cr::bf16>), grid, dim3(256), 0, 0, m, n, k, c, static_cast<const cr::bf16*>(a),
                         static_cast<const cr::bf16*>(b));
    else
      hipLaunchKernelGGL((tile_kernel<cr::f16>), grid, dim3(256), 0, 0, m, n, k, c, static_cast<const cr::f16*>(a),
                         static_cast<const cr::f16*>(b));
  });
}
