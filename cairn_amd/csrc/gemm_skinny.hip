// The skinny GEMM: m <= 16 rows of a (a decode step's tokens) against b stored n x k, K-contiguous (a weight matrix
// as a linear layer keeps it), bf16 in, f32 accumulate. At m <= 16 the work is 2 m flops per b element, far below
// the ridge of the roofline, so the kernel is built around streaming b from HBM once, evenly over the CUs: every b
// byte is read by exactly one 16-byte load, and the matrix cores do the arithmetic (v_mfma_f32_16x16x32_bf16, its 16
// rows holding a's m rows and zeros), so the vector ALUs never bound it.
//
// The columns are dealt out in equal ranges of `width` (a multiple of 8, at most 16 * GROUPS), one range a
// workgroup, so that at n = 256 width every CU streams the same bytes (n = 14336: 56 columns a CU, 3.5 MFMA column
// blocks, the last half masked). In a workgroup WAVES waves each walk their own contiguous share of k for all of its
// columns, in chunks of CH k-steps of 32: a's chunk is held in registers, and b's column blocks are loaded one at a
// time, each lane CH consecutive 16-byte pieces of its row (16 rows of CH * 64 bytes together), the next block's
// loads in flight while the current block's MFMAs run. Asking for each row's bytes together keeps DRAM pages open:
// the same loads spread over time, 64 bytes of a row at a time, measured a fifth slower. The waves' partial sums meet
// in LDS and are added in wave order, so two runs give the same bits. The reference has no decode path: its one
// tiling runs a 1 x n x k call as 64 x 64 tiles (src/cairn/runtime/cairn_tensor.hpp:206-221).
#include <hip/hip_runtime.h>
#include <algorithm>
#include <type_traits>
#include <utility>
#include "kernels.hpp"
#include "mfma.hpp"
#include "ring.hpp"

namespace cairn::gemm {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef std::uint32_t w32x4 __attribute__((ext_vector_type(4)));

__device__ inline __amdgpu_buffer_rsrc_t span(const void* base, std::int64_t bytes) {
  const std::int64_t capped = bytes < 0 ? 0 : (bytes > 0x7fffffffLL ? 0x7fffffffLL : bytes);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)capped, 0x00020000);
}
constexpr int NOWHERE = 0x7fffffff;

template<int GROUPS, int WAVES, int CH>
__global__ void __launch_bounds__(64 * WAVES) skinny_gemm(Params p, int width) {
  __shared__ f32x4 partial[WAVES][GROUPS][64];
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);  // uniform: the k loop below is a scalar loop
  const int n0 = int(blockIdx.x) * width;
  const int end = n0 + width < p.n ? n0 + width : p.n;  // this workgroup's columns: [n0, end)
  const int row = lane & 15, piece = lane >> 4;         // MFMA operand: row (of a, or column of b), 8-element k piece

  // b's rows n0 .., from their first element; a whole.
  const char* bp = static_cast<const char*>(p.b) + std::int64_t(n0) * p.ldb * 2;
  const std::int64_t bbytes = (std::int64_t(p.n - 1) * p.ldb + p.k) * 2 - std::int64_t(n0) * p.ldb * 2;
  const __amdgpu_buffer_rsrc_t rb = span(bp, bbytes);
  const __amdgpu_buffer_rsrc_t ra = span(p.a, (std::int64_t(p.m - 1) * p.lda + p.k) * 2);
  int boff[GROUPS];
#pragma unroll
  for(int g = 0; g < GROUPS; ++g)
    boff[g] = n0 + 16 * g + row < end ? int((16 * g + row) * p.ldb * 2) + 16 * piece : NOWHERE;
  const int aoff = row < p.m ? int(row * p.lda * 2) + 16 * piece : NOWHERE;

  // This wave's k-steps of 32: [first, last). Steps whole in k (below `whole`) need no per-lane test.
  const int steps = (p.k + 31) / 32, whole = p.k / 32;
  const int first = int(std::int64_t(steps) * wave / WAVES), last = int(std::int64_t(steps) * (wave + 1) / WAVES);
  f32x4 acc[GROUPS];
#pragma unroll
  for(int g = 0; g < GROUPS; ++g) acc[g] = f32x4{0, 0, 0, 0};

  // The offset of a lane's 16 bytes at `step`, or one past every range (the load reads zeros: a masked row or
  // column, a step past this wave's share, or k past its end). NOWHERE + step * 64 stays above every buffer's range.
  auto offset = [&](int base, int step) {
    int o = base + step * 64;
    if(step >= last) o = NOWHERE;  // uniform: the next wave's step, or past k
    else if(step >= whole)         // uniform: the partial last step of k
      o = step * 32 + 8 * piece < p.k && base != NOWHERE ? o : NOWHERE;
    return o;
  };
  w32x4 xa[CH], xb[2][CH];
  // A chunk of CH steps wholly inside this wave's share and inside k (every chunk but perhaps a wave's last) loads
  // with plain offsets; the other takes `offset`'s tests. CLEAN is a compile-time switch between the two copies.
  auto chunk = [&](int s0, auto clean) {
    constexpr bool CLEAN = decltype(clean)::value;
    auto at = [&](int base, int step) { return CLEAN ? (base == NOWHERE ? NOWHERE : base + step * 64) : offset(base, step); };
    auto load_b = [&](int g, int buf) {
#pragma unroll
      for(int u = 0; u < CH; ++u)
        xb[buf][u] = __builtin_bit_cast(w32x4, __builtin_amdgcn_raw_buffer_load_b128(rb, at(boff[g], s0 + u), 0, 0));
    };
    // Zeros (steps past the share read nothing) add nothing: the accumulators start at +0 and stay off -0.
    auto mfma = [&](int g, int buf) {
#pragma unroll
      for(int u = 0; u < CH; ++u)
        acc[g] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, xa[u]),
                                                         __builtin_bit_cast(bf16x8, xb[buf][u]), acc[g], 0, 0, 0);
    };
#pragma unroll
    for(int u = 0; u < CH; ++u)
      xa[u] = __builtin_bit_cast(w32x4, __builtin_amdgcn_raw_buffer_load_b128(ra, at(aoff, s0 + u), 0, 0));
    load_b(0, 0);
#pragma unroll
    for(int g = 0; g < GROUPS; ++g) {
      // Scheduling fences keep the next block's loads ahead of this block's MFMAs, which wait only for their own.
      __builtin_amdgcn_sched_barrier(0);
      if(g + 1 < GROUPS) load_b(g + 1, (g + 1) & 1);
      __builtin_amdgcn_sched_barrier(0);
      mfma(g, g & 1);
    }
    __builtin_amdgcn_sched_barrier(0);
  };
  const int clean_end = last < whole ? last : whole;  // steps below this need no test
  int s0 = first;
  for(; s0 + CH <= clean_end; s0 += CH) chunk(s0, std::true_type{});
  for(; s0 < last; s0 += CH) chunk(s0, std::false_type{});  // a short or partial last chunk

#pragma unroll
  for(int g = 0; g < GROUPS; ++g) partial[wave][g][lane] = acc[g];
  __syncthreads();
  if(wave) return;
  // Lane l holds rows 4 (l/16) .. +3 of column n0 + 16 g + l%16.
#pragma unroll
  for(int g = 0; g < GROUPS; ++g) {
    f32x4 sum = partial[0][g][lane];
#pragma unroll
    for(int w = 1; w < WAVES; ++w) sum = sum + partial[w][g][lane];
    const int n = n0 + 16 * g + (lane & 15);
    if(n >= end) continue;
#pragma unroll
    for(int r = 0; r < 4; ++r) {
      const int m = 4 * (lane >> 4) + r;
      if(m >= p.m) continue;
      float v[1] = {sum[r]};
      epilogue<1>(p, m, n, v);
      const std::int64_t at = std::int64_t(m) * p.ldc + n;
      if(p.c_type == CAIRN_TYPE_F32) {
        float* out = static_cast<float*>(p.c) + at;
        *out = p.accumulate ? *out + v[0] : v[0];
      } else {
        static_cast<std::uint16_t*>(p.c)[at] = p.c_type == CAIRN_TYPE_BF16 ? narrow_bf16(v[0]) : narrow_f16(v[0]);
      }
    }
  }
}

// The ring form (cairn_skinny says for which m and n, with which stages and widths): b's rows of the workgroup (up to
// 64) and a's 16 rows go from HBM straight into an LDS ring by `buffer_load ... lds`, KC bytes of k a row a stage, S
// stages, so that up to S - 1 stages are in flight without a register held for them, each load 1024 / KC rows x KC
// contiguous bytes. Wave w multiplies rows 16 w .. 16 w + 15 of b (the workgroup's columns) over the whole stage, so
// its accumulator is whole at the end and nothing is reduced across waves. One barrier a stage, as the GEMM ring
// (wave.hpp): past it the stage has landed for every wave and the stage before it is free for the refill.
// A row's 16-byte units are stored swizzled, unit u of row r at u ^ (r % 32), so the 16 rows an MFMA operand read
// takes are on distinct banks; the swizzle is applied by choosing which global unit each lane fetches.
// f(integral_constant<U>) for U = 0 .. N-1.
template<int N, class F> __device__ __forceinline__ void unrolled_loads(F&& f) {
  [&]<int... U>(std::integer_sequence<int, U...>) {
    (f(std::integral_constant<int, U>{}), ...);
  }(std::make_integer_sequence<int, N>{});
}

template<int S, int KC, int ROWS_B = 64>
__global__ void __launch_bounds__(256) skinny_ring(Params p, int width) {
  constexpr int ROWS_A = 16, UNITS = KC / 16, ROWS_PER_LOAD = 1024 / KC;
  constexpr int B_BYTES = ROWS_B * KC, STAGE = (ROWS_B + ROWS_A) * KC;
  constexpr int LOADS_B = ROWS_B / ROWS_PER_LOAD / 4, LOADS_A = ROWS_A / ROWS_PER_LOAD / 4;  // a wave's, a stage
  constexpr int LOADS = LOADS_B + LOADS_A;
  static_assert((KC == 256 || KC == 512 || KC == 1024) && LOADS_B % 4 == 0 && LOADS_A <= 4, "loads go out in groups of four");
  static_assert(ROWS_B % 16 == 0 && ROWS_B <= 64, "a wave multiplies 16 of b's rows");
  __shared__ __attribute__((aligned(1024))) char lds[S * STAGE];
  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  const int n0 = int(blockIdx.x) * width;                // width <= 64: the columns of this workgroup
  const int rows = p.n - n0 < width ? p.n - n0 : width;  // b's rows of this workgroup
  const unsigned ring = lds_address(lds);

  // b's rows n0 .., a's rows 0 .., each through its own range (zero fill past the last valid byte).
  Dma dma;
  const Dma::Rsrc rb = Dma::resource(static_cast<const char*>(p.b) + std::int64_t(n0) * p.ldb * 2,
                                     std::int64_t(rows - 1) * p.ldb * 2 + std::int64_t(p.k) * 2);
  const Dma::Rsrc ra = Dma::resource(static_cast<const char*>(p.a), std::int64_t(p.m - 1) * p.lda * 2 + std::int64_t(p.k) * 2);
  const int kbytes = p.k * 2, T = (kbytes + KC - 1) / KC;
  // Load j of this wave's stage (j < LOADS_B: b's rows 2 (8 w + j) + lane / 32; else a's 2 (2 w + j - LOADS_B) + ..),
  // this lane's unit: the global unit that lands at LDS position lane % 32 of its row.
  auto offset = [&](int j, int st) {
    const bool is_b = j < LOADS_B;
    const int q = is_b ? LOADS_B * wave + j : LOADS_A * wave + j - LOADS_B;  // the load's 1 KiB block of the stage
    const int r = ROWS_PER_LOAD * q + lane / UNITS, pos = lane % UNITS;
    const int u = pos ^ (r & (UNITS - 1));
    const int kb = st * KC + 16 * u;
    const bool in = kb < kbytes && (is_b ? r < rows : r < p.m);
    return in ? int(r * (is_b ? p.ldb : p.lda) * 2 + kb) : 0x7fffffff;
  };
  auto issue = [&](int st) {  // this wave's loads of stage st into buffer st % S, M0 once for each four
    const unsigned base = ring + unsigned((st % S) * STAGE);
#pragma unroll
    for(int g = 0; g < LOADS_B / 4; ++g) {
      dma.set_base(base + unsigned(LOADS_B * wave + 4 * g) * 1024u);
      dma.template load_lds_imm<0>(rb, offset(4 * g, st));
      dma.template load_lds_imm<1>(rb, offset(4 * g + 1, st));
      dma.template load_lds_imm<2>(rb, offset(4 * g + 2, st));
      dma.template load_lds_imm<3>(rb, offset(4 * g + 3, st));
    }
    dma.set_base(base + unsigned(B_BYTES) + unsigned(LOADS_A * wave) * 1024u);
    unrolled_loads<LOADS_A>([&](auto u) { dma.template load_lds_imm<decltype(u)::value>(ra, offset(LOADS_B + decltype(u)::value, st)); });
  };

  typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
  f32x4 acc = f32x4{0, 0, 0, 0};
  const int row = lane & 15, piece = lane >> 4;
  const int rb_row = 16 * wave + row;  // this lane's b row (the MFMA's column) and a row
  for(int st = 0; st < S - 1; ++st) issue(st);
  for(int st = 0; st < T; ++st) {
    wait_loads<(S - 2) * LOADS>();                   // stage st has landed (this wave's part)
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this wave's reads of stage st - 1 are done
    barrier();                                         // every wave's: stage st is whole, stage st - 1 is free
    issue(st + S - 1);                                 // into stage st - 1's buffer; past k it reads nothing
    const char* stage = lds + (st % S) * STAGE;
    if(16 * wave >= ROWS_B) continue;  // uniform: a wave past b's rows loads, and multiplies nothing
#pragma unroll
    for(int s = 0; s < KC / 64; ++s) {  // the stage's k-steps of 32 elements
      const int u = 4 * s + piece;
      const w32x4 xb = *reinterpret_cast<const w32x4*>(stage + rb_row * KC + 16 * (u ^ (rb_row & (UNITS - 1))));
      const w32x4 xa = *reinterpret_cast<const w32x4*>(stage + B_BYTES + row * KC + 16 * (u ^ row));
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, xa), __builtin_bit_cast(bf16x8, xb), acc,
                                                    0, 0, 0);
    }
  }
  wait_loads<0>();  // the loads past the last stage land before the workgroup's LDS is given back

  // Lane l holds rows 4 (l / 16) .. +3 (of a) of column n0 + 16 w + l % 16.
  if(rb_row >= rows) return;  // a column past this workgroup's (the next one's, or past n)
  const int n = n0 + rb_row;
#pragma unroll
  for(int r = 0; r < 4; ++r) {
    const int m = 4 * piece + r;
    if(m >= p.m) continue;
    float v[1] = {acc[r]};
    epilogue<1>(p, m, n, v);
    const std::int64_t at = std::int64_t(m) * p.ldc + n;
    if(p.c_type == CAIRN_TYPE_F32) {
      float* out = static_cast<float*>(p.c) + at;
      *out = p.accumulate ? *out + v[0] : v[0];
    } else {
      static_cast<std::uint16_t*>(p.c)[at] = p.c_type == CAIRN_TYPE_BF16 ? narrow_bf16(v[0]) : narrow_f16(v[0]);
    }
  }
}

// The row-streaming form, for m = 1 and 2 and k <= 4096 (a decode step's one or two tokens): a wave owns a
// contiguous run of b's rows (the output's columns), wave w of `waves` rows [w n / waves, (w + 1) n / waves), so that
// no two waves' runs differ by more than a row, and reads each row front to back, 1 KiB a load (64 lanes x 16 bytes),
// so every wave streams one contiguous region of HBM, as a plain copy does. The arithmetic is small enough for the
// vector ALUs: lane l holds a's 16-byte pieces at the same k as its pieces of b (loaded once), and v_dot2_f32_bf16
// adds two products of the packed pairs into its f32 sum an instruction (no widening of either operand), and the
// wave's 64 partial sums of a row meet in a fixed DPP pattern, so two runs give the same bits. The next row's loads
// are issued before the current row is summed: two rows of a wave in flight, KCH KiB each.
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
template<int M, int KCH, bool PLAIN, int OUT>
__global__ void __launch_bounds__(256, 3) skinny_rows(Params p, int waves) {
  const int t = threadIdx.x, lane = t & 63;
  const int wave = int(blockIdx.x) * 4 + __builtin_amdgcn_readfirstlane(t >> 6);
  const int first = int(std::int64_t(wave) * p.n / waves);
  const int last = int(std::int64_t(wave + 1) * p.n / waves);  // rows [first, last) of b
  if(first >= last) return;
  const int kbytes = p.k * 2;
  // Piece c of a row: bytes 1024 c + 16 l; past k it reads zeros.
  auto at = [&](int c) { return 1024 * c + 16 * lane < kbytes ? 1024 * c + 16 * lane : 0x7fffffff; };
  const __amdgpu_buffer_rsrc_t ra = span(p.a, (std::int64_t(M - 1) * p.lda + p.k) * 2);
  w32x4 xa[M][KCH];
#pragma unroll
  for(int i = 0; i < M; ++i)
#pragma unroll
    for(int c = 0; c < KCH; ++c) {
      const int o = at(c);
      xa[i][c] = i < p.m ? __builtin_bit_cast(w32x4, __builtin_amdgcn_raw_buffer_load_b128(
                               ra, o == 0x7fffffff ? o : int(i * p.lda * 2) + o, 0, 0))
                         : w32x4{0u, 0u, 0u, 0u};
    }
  const char* brow = static_cast<const char*>(p.b) + std::int64_t(first) * p.ldb * 2;
  const __amdgpu_buffer_rsrc_t rb = span(brow, (std::int64_t(last - first - 1) * p.ldb + p.k) * 2);
  w32x4 xb[2][KCH];
  auto load = [&](int r, w32x4 (&dst)[KCH]) {  // row first + r; past the wave's last row, zeros
#pragma unroll
    for(int c = 0; c < KCH; ++c) {
      const int o = at(c);
      dst[c] = __builtin_bit_cast(w32x4, __builtin_amdgcn_raw_buffer_load_b128(rb, o == 0x7fffffff ? o : int(r * p.ldb * 2) + o, 0, 0));
    }
  };
  auto wave_sum = [&](float v) {  // the same fixed pattern for every row: quads, half rows, rows, then the 4 rows
    v = v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
    v = v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
    v = v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
    v = v + __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false));
    const float s0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 0));
    const float s1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 16));
    const float s2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 32));
    const float s3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 48));
    return (s0 + s1) + (s2 + s3);
  };
  // The epilogue's terms of row first + r (column n of the output), where there are any (PLAIN: none, and c is not
  // read): its column scale and bias, and, for an f32 output accumulated into, the old values of c; identities (1, -0)
  // where a term is absent, which change no bit of what the stated steps give. They are fetched with the row's own
  // loads, through buffer ranges from the wave's first row (an absent term's range is empty and reads zero without
  // touching memory), so that waiting for them is waiting for the row: loaded where the epilogue needs them, after
  // the next row's loads, each wait for them would drain the prefetch (loads complete in order).
  struct Terms {
    std::uint32_t cs, b16, b32, old[M];
  };
  float rs[M];
#pragma unroll
  for(int i = 0; i < M; ++i) rs[i] = !PLAIN && p.row_scale && i < p.m ? p.row_scale[i] : 1.0f;
  const int rows = last - first;
  const bool old_c = OUT == CAIRN_TYPE_F32 && p.accumulate;
  const bool bias16 = p.bias && p.bias_type == CAIRN_TYPE_BF16, bias32 = p.bias && !bias16;
  auto range = [&](bool on, const void* base, int bytes) {
    return span(on ? base : nullptr, on ? std::int64_t(rows) * bytes : 0);
  };
  const __amdgpu_buffer_rsrc_t r_cs = range(!PLAIN && p.col_scale, p.col_scale + first, 4);
  const __amdgpu_buffer_rsrc_t r_b16 = range(!PLAIN && bias16, static_cast<const std::uint16_t*>(p.bias) + first, 2);
  const __amdgpu_buffer_rsrc_t r_b32 = range(!PLAIN && bias32, static_cast<const float*>(p.bias) + first, 4);
  __amdgpu_buffer_rsrc_t r_old[M];
#pragma unroll
  for(int i = 0; i < M; ++i)
    r_old[i] = range(!PLAIN && old_c && i < p.m, static_cast<const float*>(p.c) + std::int64_t(i) * p.ldc + first, 4);
  auto terms_of = [&](int r, Terms& v) {
    if constexpr(!PLAIN) {
      v.cs = __builtin_amdgcn_raw_buffer_load_b32(r_cs, 4 * r, 0, 0);
      v.b16 = __builtin_amdgcn_raw_buffer_load_b16(r_b16, 2 * r, 0, 0);
      v.b32 = __builtin_amdgcn_raw_buffer_load_b32(r_b32, 4 * r, 0, 0);
#pragma unroll
      for(int i = 0; i < M; ++i) v.old[i] = __builtin_amdgcn_raw_buffer_load_b32(r_old[i], 4 * r, 0, 0);
    }
  };
  // Row first + r: its sums, then the epilogue's steps in their stated order (kernels.hpp, epilogue) and the store.
  auto row = [&](int r, const w32x4 (&xr)[KCH], const Terms& tr) {
    float acc[M];
#pragma unroll
    for(int i = 0; i < M; ++i) acc[i] = 0.0f;
#pragma unroll
    for(int c = 0; c < KCH; ++c)
#pragma unroll
      for(int e = 0; e < 4; ++e) {
        // Each element goes through a scalar first: this compiler turned a bit_cast of an element of a vector
        // (xr[c][e]) into a read of element 0 whatever e was.
        const std::uint32_t wb = xr[c][e];
        const bf16x2 vb = __builtin_bit_cast(bf16x2, wb);
#pragma unroll
        for(int i = 0; i < M; ++i) {
          const std::uint32_t wa = xa[i][c][e];
          acc[i] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, wa), vb, acc[i], false);
        }
      }
    const int n = first + r;
#pragma unroll
    for(int i = 0; i < M; ++i) {
      float v = wave_sum(acc[i]);
      if(i >= p.m || lane != 0) continue;
      if constexpr(!PLAIN) {
        v = v * rs[i];
        v = v * (p.col_scale ? from_bits(tr.cs) : 1.0f);
        v = v + (bias16 ? from_bits(std::uint32_t(tr.b16) << 16) : (bias32 ? from_bits(tr.b32) : -0.0f));
        if(p.act == CAIRN_ACT_RELU) v = v < 0.0f ? 0.0f : v;
        else if(p.act == CAIRN_ACT_GELU) v = gelu(v);
      }
      const std::int64_t o = std::int64_t(i) * p.ldc + n;  // OUT is the output's type: no branch on it a row
      if constexpr(OUT == CAIRN_TYPE_F32) static_cast<float*>(p.c)[o] = !PLAIN && old_c ? from_bits(tr.old[i]) + v : v;
      else if constexpr(OUT == CAIRN_TYPE_BF16) static_cast<std::uint16_t*>(p.c)[o] = narrow_bf16(v);
      else static_cast<std::uint16_t*>(p.c)[o] = narrow_f16(v);
    }
  };
  // Two rows an iteration, so that each buffer is named at compile time; the next row's loads (and terms) go out
  // before a row is summed. Every iteration issues the loads of the row after its two, also past the wave's last
  // row, where they read zeros without touching memory: issued on one path of a branch, they would leave the wait
  // before the second row counting as if they had not been, a wait for that prefetch (measured 1-2% slower).
  Terms t0, t1;
  terms_of(0, t0);
  load(0, xb[0]);
  int r = 0;
  for(; r + 2 <= rows; r += 2) {
    terms_of(r + 1, t1);
    load(r + 1, xb[1]);
    row(r, xb[0], t0);
    terms_of(r + 2, t0);
    load(r + 2, xb[0]);
    row(r + 1, xb[1], t1);
  }
  if(r < rows) row(r, xb[0], t0);
}

// The row-streaming form's launch: its instance for m (1 or 2), the epilogue (PLAIN: no terms, c not read) and the
// output type. `lds` bytes of LDS a workgroup, which the kernel does not touch, cap the workgroups a CU holds at once
// (0: as many as the registers allow).
template<int M, bool PLAIN> hipError_t launch_rows(const Params& p, hipStream_t s, int waves, unsigned lds) {
  const dim3 grid(unsigned(waves / 4)), block(256);
  if(p.c_type == CAIRN_TYPE_BF16) hipLaunchKernelGGL((skinny_rows<M, 8, PLAIN, CAIRN_TYPE_BF16>), grid, block, lds, s, p, waves);
  else if(p.c_type == CAIRN_TYPE_F16) hipLaunchKernelGGL((skinny_rows<M, 8, PLAIN, CAIRN_TYPE_F16>), grid, block, lds, s, p, waves);
  else hipLaunchKernelGGL((skinny_rows<M, 8, PLAIN, CAIRN_TYPE_F32>), grid, block, lds, s, p, waves);
  return hipGetLastError();
}


// The streaming form, for a few rows of a (m = 2 .. 4 at the decode shape): the matrix core fed straight from
// global memory, no LDS. A wave owns 16 consecutive rows of b and all of k. Each step of 32 k is one 16-byte load of
// a (lane l: row l % 16, zero past m; chunk 4 s + l / 16), one of b (row l % 16 of the wave's 16, the same chunk)
// and one v_mfma_f32_16x16x32_bf16 into the wave's one accumulator. So each b load instruction reads 64 bytes of
// each of 16 rows: DRAM sees 16 rows streaming side by side, the pattern of the fastest pure read measured on the
// box. a, at most 16 rows, stays in the caches. D steps make a group; two groups of loads are in flight while the
// matrix core works through the one before. The accumulator's lane l, value v is row 4 (l / 16) + v of a and row
// l % 16 of the block; the k order is the matrix core's, step by step, so two runs give the same bits.
// A workgroup of four waves takes `rows` consecutive rows of b (at most 64; n = 14336: 56, one workgroup a CU).
template<int D>
__global__ void __launch_bounds__(256) skinny_stream(Params p, int rows) {
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int row0 = int(blockIdx.x) * rows + 16 * wave;
  const int left = rows - 16 * wave < p.n - row0 ? rows - 16 * wave : p.n - row0;
  const int here = left < 16 ? left : 16;  // rows of b this wave holds
  if(here <= 0) return;
  const int chunks = p.k / 8;               // 16-byte chunks of a row (k is a multiple of 8)
  const int whole = chunks / 4, steps = (chunks + 3) / 4;
  const int r = lane & 15, q = lane >> 4;
  const __amdgpu_buffer_rsrc_t ra = span(p.a, (std::int64_t(p.m - 1) * p.lda + p.k) * 2);
  const char* bb = static_cast<const char*>(p.b) + std::int64_t(row0) * p.ldb * 2;
  const __amdgpu_buffer_rsrc_t rb = span(bb, (std::int64_t(here - 1) * p.ldb + p.k) * 2);
  // Offsets at step 0; step s adds 64 s. A row past the operand's starts at NOWHERE and stays past every resource.
  const unsigned a0 = r < p.m ? unsigned(r * p.lda * 2 + q * 16) : unsigned(NOWHERE);
  const unsigned b0 = r < here ? unsigned(r * p.ldb * 2 + q * 16) : unsigned(NOWHERE);
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  w32x4 xa[2][D], xb[2][D];
  auto load = [&](int g, w32x4 (&da)[D], w32x4 (&db)[D]) {
#pragma unroll
    for(int d = 0; d < D; ++d) {
      const unsigned at = 64u * unsigned(g * D + d);
      db[d] = __builtin_bit_cast(w32x4, __builtin_amdgcn_raw_buffer_load_b128(rb, int(b0 + at), 0, 0));
      da[d] = __builtin_bit_cast(w32x4, __builtin_amdgcn_raw_buffer_load_b128(ra, int(a0 + at), 0, 0));
    }
  };
  auto mma = [&](const w32x4 (&da)[D], const w32x4 (&db)[D]) {
#pragma unroll
    for(int d = 0; d < D; ++d)
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, da[d]), __builtin_bit_cast(bf16x8, db[d]),
                                                   acc, 0, 0, 0);
  };
  const int groups = whole / D;  // groups of D whole steps
  if(groups > 0) load(0, xa[0], xb[0]);
  for(int g = 0; g < groups; g += 2) {  // two groups an iteration, so that each buffer is named at compile time
    if(g + 1 < groups) load(g + 1, xa[1], xb[1]);
    mma(xa[0], xb[0]);
    if(g + 2 < groups) load(g + 2, xa[0], xb[0]);
    if(g + 1 < groups) mma(xa[1], xb[1]);
  }
  for(int st = groups * D; st < steps; ++st) {  // the rest one step at a time; chunks past k read zeros
    const bool in = 4 * st + q < chunks;
    const unsigned at = 64u * unsigned(st);
    w32x4 a1[1], b1[1];
    b1[0] = __builtin_bit_cast(w32x4, __builtin_amdgcn_raw_buffer_load_b128(rb, in ? int(b0 + at) : NOWHERE, 0, 0));
    a1[0] = __builtin_bit_cast(w32x4, __builtin_amdgcn_raw_buffer_load_b128(ra, in ? int(a0 + at) : NOWHERE, 0, 0));
    acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a1[0]), __builtin_bit_cast(bf16x8, b1[0]),
                                                 acc, 0, 0, 0);
  }
  if(r >= here) return;
  const int n = row0 + r;
#pragma unroll
  for(int v = 0; v < 4; ++v) {
    const int i = 4 * q + v;
    if(i >= p.m) continue;
    float x[1] = {acc[v]};
    epilogue<1>(p, i, n, x);
    const std::int64_t o = std::int64_t(i) * p.ldc + n;
    if(p.c_type == CAIRN_TYPE_F32) {
      float* out = static_cast<float*>(p.c) + o;
      *out = p.accumulate ? *out + x[0] : x[0];
    } else {
      static_cast<std::uint16_t*>(p.c)[o] = p.c_type == CAIRN_TYPE_BF16 ? narrow_bf16(x[0]) : narrow_f16(x[0]);
    }
  }
}

}  // namespace cairn::gemm

// The width of a workgroup's columns for n: n spread evenly over the 256 CUs, in multiples of 8, from 8 up to the
// 64 columns a workgroup holds (past 256 x 64 columns the workgroups simply grow in number).
int cairn_skinny_width(int n) {
  const int even = (n + 255) / 256;
  const int w = (even + 7) / 8 * 8;
  return w < 8 ? 8 : (w > 64 ? 64 : w);
}

hipError_t cairn_skinny(const cairn::gemm::Params& p, hipStream_t s, int) {
  // Four forms, chosen by what measured fastest on the decode shape (n = 14336, k = 4096) in one run of each set:
  // The forms by m, each chosen side by side in one process: m = 1 and 2, whole rows a wave (below); m = 3 .. 16 from
  // n = 8193 to 16384, the half-height ring; m = 3, 4 elsewhere from n = 2048, the streaming form (m = 4 4.76 against
  // 4.58 TB/s for the register form, m = 3 4.85 against 4.74; holding a in LDS instead was slower at every m); m = 5 ..
  // 16 from n = 4096, the 256-byte ring (4.6 against 4.4 TB/s for the register form at m = 16, and 4.0 for the
  // streaming form, whose loads of a's 16 rows double the L2 traffic); otherwise the register form.
  // Whole rows a wave, dealt evenly, on packed bf16 dot products, for m = 1 from n = 2048 and m = 2 from n = 4096.
  // m = 1: 8192 waves from n = 8192, 4096 from 4096, else 2048, at most four workgroups a CU (72 registers would let
  // seven share one; the LDS asked for leaves room for four). Side by side at k = 4096 (TB/s) against the form before
  // (f32 FMAs on operands widened in registers, 165 registers: 12 waves a CU): n = 8192 6.04-6.05 against 5.66-5.68,
  // 14336 5.76-5.78 against 5.49-5.54, 16384 5.72-5.75 against 5.55-5.66, 28672 5.89-5.90 against 5.88-5.91; without
  // the cap 5.62, 5.69 and 5.74 at 14336, 16384 and 28672, with three workgroups a CU 5.68, 5.75, 5.92.
  // m = 2 (134 registers: three workgroups a CU): 8192 waves from n = 16384, 4096 from 8192, else 2048; against the
  // forms it replaced (the half-height ring from 8193, the streaming form below): n = 4096 4.44 against 3.21, 8192
  // 5.46 against 5.06-5.13, 11008 5.03-5.05 against 4.85-5.01, 14336 5.37-5.38 against 5.25-5.28, 16384 5.45 against
  // 4.74, 28672 5.87 against 5.07. m = 4 in this form (198 registers) ran 4.86 against the ring's 5.17-5.19.
  const int row_waves = p.m == 1 ? (p.n >= 8192 ? 8192 : (p.n >= 4096 ? 4096 : 2048))
                                 : (p.n >= 16384 ? 8192 : (p.n >= 8192 ? 4096 : 2048));
  const int most = (p.n + row_waves - 1) / row_waves;  // rows the busiest wave streams
  if(((p.m == 1 && p.n >= 2048) || (p.m == 2 && p.n >= 4096)) && p.k <= 4096 &&
     std::int64_t(most + 1) * p.ldb * 2 < 0x7f000000LL) {
    const bool plain = !p.row_scale && !p.col_scale && !p.bias && p.act == CAIRN_ACT_NONE &&
                       !(p.c_type == CAIRN_TYPE_F32 && p.accumulate);
    constexpr unsigned FOUR = 160u * 1024 / 5 + 64;  // of the CU's 160 KiB of LDS: room for four workgroups, not five
    if(p.m == 1)
      return plain ? cairn::gemm::launch_rows<1, true>(p, s, row_waves, FOUR)
                   : cairn::gemm::launch_rows<1, false>(p, s, row_waves, FOUR);
    return plain ? cairn::gemm::launch_rows<2, true>(p, s, row_waves, 0) : cairn::gemm::launch_rows<2, false>(p, s, row_waves, 0);
  }
  // The half-height ring: three 512-byte stages of 32 rows of b (72 KiB of LDS, two workgroups a CU), n dealt to
  // 512 workgroups, for m >= 2 from n = 8193 to 16384 and for m > 4 from n = 7681. A load brings two rows' 512
  // contiguous bytes instead of four rows' 256, and each CU keeps two workgroups' stages in flight. Side by side over
  // n = 8192 .. 16384 and m = 2, 4, 8, 16 (k = 4096, TB/s): n = 14336 5.12-5.19 against 4.83-4.91 for the form
  // chosen before (three 512-byte stages of 56 rows, one workgroup a CU), n = 12288 4.94-5.06 against 4.72-4.83,
  // n = 11008 4.77-4.97 against 4.57-4.67, n = 16384 4.64-4.71 against 4.33-4.63; at n = 8192 m = 8, 16 4.15-4.24
  // against 3.91-4.07, m = 2, 4 1% behind the streaming form. A width rounded up to 8 (448 workgroups at
  // n = 14336) left CUs with one workgroup: far slower.
  const int even = cairn_skinny_width(p.n);
  const int half = (p.n + 511) / 512;  // columns a workgroup, 512 workgroups
  if(p.m >= 2 && half <= 32 && (half > 16 || (p.m > 4 && half == 16))) {
    hipLaunchKernelGGL((cairn::gemm::skinny_ring<3, 512, 32>), dim3(unsigned((p.n + half - 1) / half)), dim3(256), 0,
                       s, p, half);
    return hipGetLastError();
  }
  if(p.m >= 2 && p.m <= 4 && p.n >= 2048) {  // rows of b a workgroup: n over the 256 CUs, 16 .. 64
    const int even = (p.n + 255) / 256;
    // 32 rows (n about 8192) leave two of a workgroup's four waves idle: 16 rows, two workgroups a CU, measured 4.26
    // against 3.24 TB/s there (m = 4, n = 8192); at the other widths tried (4096 .. 14336) this rule was best or even.
    const int fit = std::min(64, std::max(16, (even + 7) / 8 * 8));
    const int rows = fit == 32 ? 16 : fit;
    hipLaunchKernelGGL((cairn::gemm::skinny_stream<8>), dim3(unsigned((p.n + rows - 1) / rows)), dim3(256), 0, s, p,
                       rows);
    return hipGetLastError();
  }
  if(p.m > 4 && p.n >= 4096) {
    // The ring with 256-byte stages (80 KiB of LDS, so two workgroups share a CU where there are more than 256), below
    // n = 7681 and above 16384 (between them the half-height ring above). Columns a workgroup: 32 below n = 8192
    // (128 .. 224 workgroups), 64 above. Measured side by side on two boxes at m = 5 .. 16 against the 512-byte ring
    // (64 columns, 160 KiB) and the register form: 9-19% faster at n = 5120 .. 7168 and 2-15% from 16384 on, where two
    // workgroups a CU keep every CU streaming.
    const int width = p.n < 8192 ? 32 : (even >= 56 ? even : 64);
    hipLaunchKernelGGL((cairn::gemm::skinny_ring<4, 256>), dim3(unsigned((p.n + width - 1) / width)), dim3(256), 0, s,
                       p, width);
    return hipGetLastError();
  }
  constexpr int GROUPS = 4, WAVES = 4, CH = 8;  // measured best of 2 / 4 / 8 waves and chunks of 8 / 16 steps
  const int width = cairn_skinny_width(p.n);
  const dim3 grid(unsigned((p.n + width - 1) / width));
  hipLaunchKernelGGL((cairn::gemm::skinny_gemm<GROUPS, WAVES, CH>), grid, dim3(64 * WAVES), 0, s, p, width);
  return hipGetLastError();
}
