// Matrix-core fragments for gfx950: one wave's operand A, operand B or accumulator of one MFMA shape, and what a wave
// does with them: fill, load through a layout, multiply-accumulate, store through a layout, and read or write one
// value of its own share. The operations and their spellings are the ones CAIRN emits for fragment code
// (src/cairn/compiler/device/fragments.py:330-405: filled, loaded, multiplied, stored, get, set), over a family of
// its own beside the reference's WMMA and mma.sync ones (src/cairn/runtime/cairn_fragment.hpp:1-294): MfmaFragment.
//
// A fragment is a wave-uniform value: all 64 lanes of a wave name the same matrix and run each operation on it
// together (with every lane active). The shapes and their instructions:
//
//   M x N x K      operands     accumulator   instruction
//   32 x 32 x 16   f16, bf16    f32           v_mfma_f32_32x32x16_{f16,bf16}
//   16 x 16 x 32   f16, bf16    f32           v_mfma_f32_16x16x32_{f16,bf16}
//   32 x 32 x 32   int8         int32         v_mfma_i32_32x32x32_i8
//
// A is M x K, B is K x N, the accumulator M x N. On the device a lane holds M * K / 64 consecutive k values of one
// row of A (row l % M, from k = (M * K / 64) * (l / M)) and the same k values of one column of B (column l % N); of
// the accumulator it holds M * N / 64 values, value v of lane l being
//
//   32 x 32:  element (8 (v / 4) + 4 (l / 32) + v % 4, l % 32)
//   16 x 16:  element (4 (l / 16) + v, l % 16)
//
// which `holder` and `element` state for the host. Each multiply-accumulate adds every product, exact in f32 (or in
// int32), to its output, the partial sums of f16/bf16 rounded to f32 in an order the hardware picks: the contract of
// mma_unordered. On the host every lane holds each fragment whole, widened exactly; a multiply adds in increasing k,
// so host code built of fragments gives, bit for bit, what the reference loop gives; and a store writes only the
// elements the lane holds on the device, so a wave's 64 lanes write each element once between them.
#pragma once
#include <cstddef>
#include <cstdint>
#include <type_traits>
#include "cairn_float.hpp"
#include "cairn_runtime.hpp"

namespace cr::frag {

enum class Role { a, b, acc };

template<Role R, int M, int N, int K> struct Shape {
  static constexpr int rows = R == Role::b ? K : M;
  static constexpr int cols = R == Role::a ? K : N;
  static constexpr int size = rows * cols;
};

constexpr unsigned WAVE = 64;

// The shapes the family has for an operand type.
template<class T, int M, int N, int K>
constexpr bool mfma_shape = std::is_same_v<T, std::int8_t>
                                ? (M == 32 && N == 32 && K == 32)
                                : (std::is_same_v<T, cr::f16> || std::is_same_v<T, cr::bf16>) &&
                                      ((M == 32 && N == 32 && K == 16) || (M == 16 && N == 16 && K == 32));

// What an operand type accumulates in, and what a whole fragment of it holds on the host: int8 into int32, the
// 16-bit floats into f32 (each widened exactly).
template<class T> using held_t = std::conditional_t<std::is_integral_v<T>, std::int32_t, float>;

// The accumulator's lane share (see above): how many values a lane holds, and which element value v of lane l is.
template<int M, int N> constexpr int values = M * N / int(WAVE);
template<int M, int N> CR_HD constexpr std::size_t row_of(unsigned lane, std::size_t v) noexcept {
  static_assert(M == N && (M == 32 || M == 16));
  return M == 32 ? 8 * (v / 4) + 4 * ((lane % WAVE) / 32) + v % 4 : 4 * ((lane % WAVE) / 16) + v;
}
template<int M, int N> CR_HD constexpr std::size_t col_of(unsigned lane) noexcept { return (lane % WAVE) % N; }
// The row-major index, in a whole fragment, of lane l's value v.
template<int M, int N> CR_HD constexpr std::size_t element(unsigned lane, std::size_t v) noexcept {
  return row_of<M, N>(lane, v) * N + col_of<M, N>(lane);
}
// The lane that holds element (r, c) of an accumulator on the device.
template<int M, int N> CR_HD constexpr unsigned holder(std::size_t r, std::size_t c) noexcept {
  static_assert(M == N && (M == 32 || M == 16));
  return M == 32 ? unsigned(c % 32 + 32 * ((r / 4) % 2)) : unsigned(c % 16 + 16 * (r / 4));
}

// ---------------------------------------------------------------------------------------------------------------
// The host: every lane holds the whole fragment.

template<Role R, class T, int M, int N, int K> struct Whole {
  static_assert(R == Role::acc || mfma_shape<T, M, N, K>, "an MFMA operand shape: 32x32x16 or 16x16x32, int8 32x32x32");
  using E = held_t<T>;
  E e[Shape<R, M, N, K>::size];
};

template<class S> CR_HD inline auto widen(const S& x) noexcept {
  if constexpr(std::is_integral_v<S>) return std::int32_t(x);
  else if constexpr(std::is_same_v<S, float>) return x;
  else return static_cast<float>(x);  // a storage float, exactly
}

template<Role R, class T, int M, int N, int K, class V> CR_HD void fill(Whole<R, T, M, N, K>& f, V x) noexcept {
  for(auto& v : f.e) v = typename Whole<R, T, M, N, K>::E(x);
}

template<Role R, class T, int M, int N, int K, class S, class At>
CR_HD void load(Whole<R, T, M, N, K>& f, const S* base, At at) noexcept {
  using F = Shape<R, M, N, K>;
  for(int r = 0; r < F::rows; ++r)
    for(int c = 0; c < F::cols; ++c) f.e[r * F::cols + c] = widen(base[at(std::size_t(r), std::size_t(c))]);
}

// d + a * b: every product exact, then added to its output in increasing k, each f32 sum rounded (int32 sums wrap,
// as the hardware's do).
template<class T, class U, int M, int N, int K>
CR_HD void mma(Whole<Role::acc, U, M, N, K>& d, const Whole<Role::a, T, M, N, K>& a,
               const Whole<Role::b, T, M, N, K>& b) noexcept {
  static_assert(std::is_same_v<held_t<T>, held_t<U>>, "int8 accumulates in int32, the 16-bit floats in f32");
  for(int i = 0; i < M; ++i)
    for(int p = 0; p < K; ++p) {
      const auto x = a.e[i * K + p];
      for(int j = 0; j < N; ++j) {
        if constexpr(std::is_integral_v<held_t<T>>)
          d.e[i * N + j] = std::int32_t(std::uint32_t(d.e[i * N + j]) + std::uint32_t(x * b.e[p * N + j]));
        else d.e[i * N + j] = d.e[i * N + j] + x * b.e[p * N + j];
      }
    }
}

template<class U, int M, int N, int K, class D, class At>
CR_HD void store(const Whole<Role::acc, U, M, N, K>& f, D* base, At at, unsigned lane) noexcept {
  for(int r = 0; r < M; ++r)
    for(int c = 0; c < N; ++c)
      if(holder<M, N>(std::size_t(r), std::size_t(c)) == lane % WAVE)
        base[at(std::size_t(r), std::size_t(c))] = D(f.e[r * N + c]);
}

// ---------------------------------------------------------------------------------------------------------------
// The device: the registers an MFMA instruction reads and writes.

#if defined(__HIP_DEVICE_COMPILE__)
template<class E, int V> using vec __attribute__((ext_vector_type(V))) = E;

template<Role R, class T, int M, int N, int K> struct Mfma;
template<class T, int M, int N, int K> struct Mfma<Role::a, T, M, N, K> {
  static_assert(mfma_shape<T, M, N, K>, "an MFMA operand shape: 32x32x16 or 16x16x32, int8 32x32x32");
  vec<std::uint32_t, 4> r;  // 16 bytes: 8 halves, or 16 int8
};
template<class T, int M, int N, int K> struct Mfma<Role::b, T, M, N, K> {
  static_assert(mfma_shape<T, M, N, K>, "an MFMA operand shape: 32x32x16 or 16x16x32, int8 32x32x32");
  vec<std::uint32_t, 4> r;
};
template<class U, int M, int N, int K> struct Mfma<Role::acc, U, M, N, K> {
  vec<held_t<U>, values<M, N>> c;
};

__device__ inline unsigned lane() { return __lane_id(); }

// The 16-bit pattern or byte of one operand element.
template<class S> __device__ inline std::uint32_t bits_of(const S& x) {
  if constexpr(std::is_integral_v<S>) return std::uint32_t(std::uint8_t(x));
  else return std::uint32_t(x.bits);
}

// A lane's operand run: KL consecutive k values of row l % M (A) or column l % N (B), element by element through
// any layout, from global memory or LDS; or, where the layout is affine with the run contiguous (an A tile stored
// by rows, a B tile by columns: `ld` nonzero and `rows` saying which) and the run starts on 16 bytes, as one
// 16-byte load.
template<Role R, class T, int M, int N, int K, class S, class At>
__device__ void load(Mfma<R, T, M, N, K>& f, const S* base, At at, std::size_t ld = 0, bool rows = true) {
  static_assert(R != Role::acc);
  constexpr int G = R == Role::a ? M : N, KL = G * K / int(WAVE);
  constexpr int BITS = std::is_integral_v<T> ? 8 : 16, PER = 32 / BITS;  // bits of an element, elements a word
  static_assert(KL * BITS == 128, "a lane's run is 16 bytes");
  const unsigned l = lane();
  const std::size_t line = l % G, k0 = std::size_t(KL) * (l / G);
  const std::size_t first = R == Role::a ? at(line, k0) : at(k0, line);
  const bool contiguous = ld != 0 && (R == Role::a ? rows : !rows);
  if(contiguous && reinterpret_cast<std::uintptr_t>(base + first) % 16 == 0) {
    f.r = *reinterpret_cast<const vec<std::uint32_t, 4>*>(base + first);
    return;
  }
  f.r = vec<std::uint32_t, 4>{0u, 0u, 0u, 0u};
#pragma unroll
  for(int e = 0; e < KL; ++e) {
    const std::size_t o = R == Role::a ? at(line, k0 + e) : at(k0 + e, line);
    f.r[e / PER] |= bits_of(base[o]) << (BITS * (e % PER));
  }
}

template<class U, int M, int N, int K, class D, class At>
__device__ void load(Mfma<Role::acc, U, M, N, K>& f, const D* base, At at, std::size_t = 0, bool = true) {
  const unsigned l = lane();
#pragma unroll
  for(int v = 0; v < values<M, N>; ++v) f.c[v] = held_t<U>(base[at(row_of<M, N>(l, v), col_of<M, N>(l))]);
}

template<Role R, class T, int M, int N, int K, class V> __device__ void fill(Mfma<R, T, M, N, K>& f, V x) {
  static_assert(R == Role::acc, "operands are loaded, not filled");
#pragma unroll
  for(int v = 0; v < values<M, N>; ++v) f.c[v] = held_t<T>(x);
}

template<class T, class U, int M, int N, int K>
__device__ void mma(Mfma<Role::acc, U, M, N, K>& d, const Mfma<Role::a, T, M, N, K>& a,
                    const Mfma<Role::b, T, M, N, K>& b) {
  static_assert(std::is_same_v<held_t<T>, held_t<U>>, "int8 accumulates in int32, the 16-bit floats in f32");
  if constexpr(std::is_same_v<T, std::int8_t>) {
    d.c = __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(vec<int, 4>, a.r), __builtin_bit_cast(vec<int, 4>, b.r),
                                                d.c, 0, 0, 0);
  } else if constexpr(std::is_same_v<T, cr::bf16>) {
    using X = vec<__bf16, 8>;
    if constexpr(M == 32)
      d.c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(X, a.r), __builtin_bit_cast(X, b.r), d.c, 0, 0, 0);
    else
      d.c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(X, a.r), __builtin_bit_cast(X, b.r), d.c, 0, 0, 0);
  } else {
    using X = vec<_Float16, 8>;
    if constexpr(M == 32)
      d.c = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(X, a.r), __builtin_bit_cast(X, b.r), d.c, 0, 0, 0);
    else
      d.c = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(X, a.r), __builtin_bit_cast(X, b.r), d.c, 0, 0, 0);
  }
}

template<class U, int M, int N, int K, class D, class At>
__device__ void store(const Mfma<Role::acc, U, M, N, K>& f, D* base, At at) {
  const unsigned l = lane();
#pragma unroll
  for(int v = 0; v < values<M, N>; ++v) {
    const held_t<U> x = f.c[v];  // through a scalar: this compiler's bit casts of a vector element misread it
    base[at(row_of<M, N>(l, v), col_of<M, N>(l))] = D(x);
  }
}
#endif

// ---------------------------------------------------------------------------------------------------------------
// What CAIRN's fragment lowering emits, with the Mfma family's name in place of Wmma or Mma.

#if defined(__HIP_DEVICE_COMPILE__)
template<Role R, class T, int M, int N, int K> using MfmaFragment = Mfma<R, T, M, N, K>;
#else
template<Role R, class T, int M, int N, int K> using MfmaFragment = Whole<R, T, M, N, K>;
#endif

template<class F, class V> CR_HD F filled(V x) noexcept {
  F f;
  fill(f, x);
  return f;
}

// `ld` and `rows` are the layout's leading dimension and orientation where it is affine, which the device's
// contiguous-run load reads; `shared` (the tile is a block's LDS array) changes nothing here: LDS and global memory
// take the same loads.
template<class F, class S, class At> CR_HD F loaded(const S* base, At at, std::size_t ld, bool rows, bool shared) noexcept {
  F f;
  (void)shared;
#if defined(__HIP_DEVICE_COMPILE__)
  load(f, base, at, ld, rows);
#else
  (void)ld, (void)rows;
  load(f, base, at);
#endif
  return f;
}

// Value v of lane l's share of an accumulator, the element (row_of, col_of) above; an index past the share traps.
// On the host the lane reads and writes that element of its whole copy: the one element of it the lane stores.
template<class U, int M, int N, int K>
CR_HD held_t<U> get(const Whole<Role::acc, U, M, N, K>& f, std::size_t v, unsigned lane) noexcept {
  if(v >= std::size_t(values<M, N>)) trap();
  return f.e[element<M, N>(lane, v)];
}
template<class U, int M, int N, int K, class V>
CR_HD Whole<Role::acc, U, M, N, K> set(Whole<Role::acc, U, M, N, K> f, std::size_t v, V x, unsigned lane) noexcept {
  if(v >= std::size_t(values<M, N>)) trap();
  f.e[element<M, N>(lane, v)] = held_t<U>(x);
  return f;
}
#if defined(__HIP_DEVICE_COMPILE__)
template<class U, int M, int N, int K>
__device__ held_t<U> get(const Mfma<Role::acc, U, M, N, K>& f, std::size_t v, unsigned) noexcept {
  if(v >= std::size_t(values<M, N>)) trap();
  return f.c[v];
}
template<class U, int M, int N, int K, class V>
__device__ Mfma<Role::acc, U, M, N, K> set(Mfma<Role::acc, U, M, N, K> f, std::size_t v, V x, unsigned) noexcept {
  if(v >= std::size_t(values<M, N>)) trap();
  f.c[v] = held_t<U>(x);
  return f;
}
#endif

template<class D, class A, class B> CR_HD D multiplied(D d, const A& a, const B& b) noexcept {
  mma(d, a, b);
  return d;
}

template<class F, class D, class At>
CR_HD void stored(const F& f, D* base, At at, std::size_t ld, bool rows, unsigned lane) noexcept {
  (void)ld, (void)rows;
#if defined(__HIP_DEVICE_COMPILE__)
  (void)lane;
  store(f, base, at);
#else
  store(f, base, at, lane);
#endif
}

}  // namespace cr::frag
