// The one-wave-a-SIMD MFMA GEMM for gfx950: four waves per workgroup, each feeding its SIMD's matrix core without a
// partner wave, with the LDS reads of its next MFMA k-step and the loads of a later stage issued between its MFMAs.
//
// A workgroup of 256 threads computes one BM x BN output tile (256 x 256 by default); wave w holds the (BM/2) x
// (BN/2) block at wave_origin (pipe.hpp), 4 x 4 blocks of 32 x 32 accumulators at 256 x 256, which live in the
// accumulation registers. The operand stages are pipe.hpp's: 64 bytes of k of every operand row a stage, STAGES deep,
// filled by buffer_load ... lds, with its swizzles and fragment reads; all four waves load both operands, a quarter
// each.
//
// Compared with eight waves of (BM/2) x (BN/4), a wave's larger block reads a third less from LDS for the same MFMA
// work (a stage is read 2 + 2 times, not 4 + 2), and the workgroup meets at one barrier a stage instead of two.
//
// Iteration `it` works on stage it in two MFMA k-steps, the operands double-buffered in registers:
//   k-step 0: the 16 MFMAs of (it, 0), between them the fragment reads of (it, 1) and b's loads of stage
//             it + STAGES - 1;
//             wait for this wave's LDS reads and for its loads of stage it + 1; barrier;
//   k-step 1: the 16 MFMAs of (it, 1), between them the fragment reads of (it + 1, 0) and a's loads of stage
//             it + STAGES, into the buffer stage it used.
// The barrier orders both hazards of the ring. Past it every wave's loads of stage it + 1 have landed (each waited
// for its own), and every wave's reads of stage it are complete (each waited for its own LDS reads, and its last reads
// of stage it were those of (it, 1)): so stage it's buffer is free from then on, and its refill is spread over the
// next 32 MFMAs, one 16-byte load a lane every fourth MFMA. A wave's loads of one operand's stage fill consecutive
// KiB of LDS (pipe.hpp, slot), so M0 is written once per operand and stage and each load picks its KiB with its
// immediate offset: a write of M0 waits for the wave's previous LDS load to leave the queue, and one per load cost a
// quarter of the loop (measured). The host runs this kernel only where no lane's offset register would go below zero
// (Loader::imm_fits).
// Every iteration issues its loads, so the loop has no branches and the wait for stage it + 1 is the same count every
// time: past the last stage they land in a buffer no later stage reads, from inside the operand's panel or (past its
// end) as zeros. Iterations come in two forms. Steady ones load stages that end at or before k (and, where k is a
// whole number of stages, those past the last) with no per-chunk k check; they run STAGES at a time, unrolled, so
// that each one's ring slot, and with it every LDS address and M0 value, is a constant. The iterations that load the
// last, partial stage check each chunk against k. The buffer resources are walked a stage at a time by scalar adds
// (pipe.hpp, Walk) in issue slots no LDS read uses, so that between two MFMAs the wave has no more to issue than the
// MFMA's 32 cycles take (tests/test_isa.py prices the compiled loop).
// Scheduling fences keep the interleave as written and keep everything on its side of the barrier.
// No atomics: the result's bits do not depend on timing.
//
// The instances (gemm_wave_<type>.hip, one file an operand type so they compile in parallel) are listed in
// wave_<type>.inc; capi.cpp's kernel table reads the same lists through wave_instances.inc.
#pragma once
#include <hip/hip_runtime.h>
#include <type_traits>
#include <utility>
#include "epilogue.hpp"
#include "kernels.hpp"
#include "mfma.hpp"
#include "pipe.hpp"
#include "ring.hpp"
#include "tile.hpp"

namespace cairn::gemm {
using namespace cairn::pipe;

// f(integral_constant<I>) for I = 0 .. N-1, in order.
template<int N, class F> __device__ __forceinline__ void unrolled(F&& f) {
  [&]<int... I>(std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
  }(std::make_integer_sequence<int, N>{});
}

// No instruction is scheduled across this point.
__device__ __forceinline__ void fence() { __builtin_amdgcn_sched_barrier(0); }

// The walk's registers as if rewritten here: the compiler cannot compute a later stage's resource from an earlier one
// ahead of time (which gathers the scalar work of an unrolled loop into one gap between MFMAs).
__device__ __forceinline__ void pin(Walk& w) { asm volatile("" : "+s"(w.at), "+s"(w.left)); }

__device__ __forceinline__ void fenced_barrier() {
  fence();
  asm volatile("s_barrier" ::: "memory");
  fence();
}

// The epilogue of a wave's accumulators, after the main loop (every wave past its last LDS read of the ring): block
// (i, j) of the wave, quad q of lane l is row m, columns n .. n+3. A bf16 output of a tile wholly inside c goes
// through LDS so that every store writes whole rows; a plain one (no scales, bias or activation) skips the
// epilogue's identity steps. Everything else takes finish's quad-by-quad stores.
// The epilogue terms of a tile, one row scale, column scale and bias a thread (thread t: row row0 + t, column
// col0 + t), loaded at the kernel's start so that their latency hides behind the main loop; the staged store reads
// them back from LDS. Identities (1, 1, -0) where a term is absent or out of range.
struct Terms {
  float rs = 1.0f, cs = 1.0f, bs = -0.0f;
};

template<class Sh>
__device__ __forceinline__ Terms prefetch_terms(const Params& p, int row0, int col0, int t) {
  static_assert(Sh::BM == 256 && Sh::BN == 256, "a thread a row and a column of the tile");
  Terms v;
  const bool staged = p.c_type == CAIRN_TYPE_BF16 && p.rows16 && row0 + Sh::BM <= p.m && col0 + Sh::BN <= p.n;
  if(!staged) return v;  // uniform; the other stores read their terms themselves
  if(p.row_scale) v.rs = p.row_scale[row0 + t];
  if(p.col_scale) v.cs = p.col_scale[col0 + t];
  if(p.bias)
    v.bs = p.bias_type == CAIRN_TYPE_BF16 ? widen_bf16(static_cast<const std::uint16_t*>(p.bias)[col0 + t])
                                          : static_cast<const float*>(p.bias)[col0 + t];
  return v;
}

template<class Sh, bool RAW, class Acc, int FM, int FN>
__device__ __forceinline__ void store_tile(const Params& p, const Acc (&acc)[FM][FN], char* lds, float* terms,
                                           const Terms& mine_terms, int wave, int row0, int col0, int wr, int wc,
                                           int lane) {
  constexpr int S = Sh::STAGES;
  const bool plain = !p.row_scale && !p.col_scale && !p.bias && p.act == CAIRN_ACT_NONE;
  const bool whole = row0 + Sh::BM <= p.m && col0 + Sh::BN <= p.n;
  if constexpr(!RAW) {
    if(p.c_type == CAIRN_TYPE_BF16 && whole && p.rows16) {  // rows of c on 16 bytes: the staged 16-byte stores
      // The wave's WTM x WTN bf16 block goes into its own part of the ring (free once every wave has passed the
      // barrier), 8 bytes a quad, then comes back 16 bytes a lane, a row of the block per 16 lanes. The 8-byte unit u
      // of row r sits at unit u ^ (r % 32) of the row, which keeps both the writes (32 rows, one unit each) and the
      // reads (16 units of one row) on distinct banks; a read of an odd row finds its two halves swapped.
      static_assert(Sh::WTN * 2 == 256 && Sh::WTM * 256 * Sh::WAVES <= S * Sh::STAGE, "a row of the block is 256 bytes");
      fenced_barrier();  // every wave is past its last read of the ring
      if(!plain) {       // uniform
        const int t = 64 * wave + lane;
        terms[t] = mine_terms.rs;
        terms[256 + t] = mine_terms.cs;
        terms[512 + t] = mine_terms.bs;
        fenced_barrier();
      }
      char* mine = lds + wave * (Sh::WTM * 256);
      const int h = lane >> 5;
      auto put = [&](int i, int j, int q, float v0, float v1, float v2, float v3) {
        const int r = 32 * i + (lane & 31);
        u32x2 w;
        w[0] = narrow2_bf16(v0, v1);
        w[1] = narrow2_bf16(v2, v3);
        const int unit = (8 * j + 2 * q + h) ^ (r & 31);
        *reinterpret_cast<u32x2*>(mine + r * 256 + unit * 8) = w;
      };
      // The rows go out as non-temporal stores: c is written once and not read again by this launch, and streaming it
      // past L2 leaves less to write back when the launch ends (4096^3: 0.5-1 us of 105 bf16, 0.7 of 63 int8 W8A8,
      // side by side against plain stores). The block goes out 32 rows at a time: group i's values are converted
      // (and go through the epilogue's steps) into LDS, then read back and stored, so that the next group's
      // arithmetic runs while this group's stores drain (a 4096^3 launch's stores take about 4 us, bound by the
      // write bandwidth of the XCDs; the dequant and GELU work before them was serial).
      const int cl = lane & 15;
      char* out = static_cast<char*>(p.c) + (std::int64_t(row0 + wr) * p.ldc + col0 + wc) * 2 + 16 * cl;
      auto emit = [&](int i) {  // rows 32 i .. 32 i + 31 of the block, 16 bytes a lane, four rows a read
#pragma unroll
        for(int s = 8 * i; s < 8 * i + 8; ++s) {
          const int r = 4 * s + (lane >> 4);
          u32x4 v = *reinterpret_cast<const u32x4*>(mine + r * 256 + 16 * (cl ^ ((r & 31) >> 1)));
          if(r & 1) v = u32x4{v[2], v[3], v[0], v[1]};
          __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(out + std::int64_t(r) * p.ldc * 2));
        }
      };
      static_assert(Sh::WTM == 32 * FM, "a group of 32 rows a block row");
      if(plain) {
#pragma unroll
        for(int i = 0; i < FM; ++i) {
#pragma unroll
          for(int j = 0; j < FN; ++j)
#pragma unroll
            for(int q = 0; q < 4; ++q)
              put(i, j, q, float(acc[i][j][4 * q]), float(acc[i][j][4 * q + 1]), float(acc[i][j][4 * q + 2]),
                  float(acc[i][j][4 * q + 3]));
          emit(i);
          fence();
        }
      } else {
        with_form(p, [&](auto form) {
          using F = decltype(form);
          float rs[FM];
#pragma unroll
          for(int i = 0; i < FM; ++i) rs[i] = terms[wr + 32 * i + (lane & 31)];
          auto col_terms = [&](int j, float (&cs)[4][4], float (&bs)[4][4]) {  // the lane's columns of block column j
#pragma unroll
            for(int q = 0; q < 4; ++q)
#pragma unroll
              for(int e = 0; e < 4; ++e) {
                const int n = wc + 32 * j + 8 * q + 4 * h + e;
                cs[q][e] = terms[256 + n];
                bs[q][e] = terms[512 + n];
              }
          };
          auto convert = [&](int i, int j, const float (&cs)[4][4], const float (&bs)[4][4]) {
#pragma unroll
            for(int q = 0; q < 4; ++q) {
              float v[4];
#pragma unroll
              for(int e = 0; e < 4; ++e) v[e] = apply<F>(float(acc[i][j][4 * q + e]), rs[i], cs[q][e], bs[q][e]);
              put(i, j, q, v[0], v[1], v[2], v[3]);
            }
          };
          constexpr bool integer = std::is_integral_v<std::remove_cvref_t<decltype(acc[0][0][0])>>;
          if constexpr(F::scaled && integer) {
            // The W8A8 dequant (int8 accumulators, scales): grouped as well, each block column's terms read from
            // LDS again for every group (held for all groups at once, they spilled registers).
#pragma unroll
            for(int i = 0; i < FM; ++i) {
#pragma unroll
              for(int j = 0; j < FN; ++j) {
                float cs[4][4], bs[4][4];
                col_terms(j, cs, bs);
                convert(i, j, cs, bs);
              }
              emit(i);
              fence();
            }
          } else if constexpr(F::scaled) {
            // Scales on float accumulators: block column by block column, then the stores (grouped, this form's
            // code made the compiler spill accumulators to scratch after the main loop of every launch).
#pragma unroll
            for(int j = 0; j < FN; ++j) {
              float cs[4][4], bs[4][4];
              col_terms(j, cs, bs);
#pragma unroll
              for(int i = 0; i < FM; ++i) convert(i, j, cs, bs);
            }
#pragma unroll
            for(int i = 0; i < FM; ++i) emit(i);
          } else {
            // Bias and an activation, no scales (the MLP forward's bias + GELU, the longest arithmetic of the
            // epilogue): grouped, every block column's biases held.
            float cs[FN][4][4], bs[FN][4][4];
#pragma unroll
            for(int j = 0; j < FN; ++j) col_terms(j, cs[j], bs[j]);
#pragma unroll
            for(int i = 0; i < FM; ++i) {
#pragma unroll
              for(int j = 0; j < FN; ++j) convert(i, j, cs[j], bs[j]);
              emit(i);
              fence();
            }
          }
        });
      }
      return;
    }
    if(plain && p.c_type == CAIRN_TYPE_BF16) {  // an edge tile: quad by quad, each checked
      char* c = static_cast<char*>(p.c);
#pragma unroll
      for(int i = 0; i < FM; ++i)
#pragma unroll
        for(int j = 0; j < FN; ++j)
#pragma unroll
          for(int q = 0; q < 4; ++q) {
            const int m = row0 + wr + 32 * i + cairn::tile::acc_m(lane);
            const int n = col0 + wc + 32 * j + cairn::tile::acc_n(lane, q);
            if(!(m < p.m && n < p.n)) continue;
            u32x2 w;
            w[0] = narrow2_bf16(float(acc[i][j][4 * q]), float(acc[i][j][4 * q + 1]));
            w[1] = narrow2_bf16(float(acc[i][j][4 * q + 2]), float(acc[i][j][4 * q + 3]));
            *reinterpret_cast<u32x2*>(c + (std::int64_t(m) * p.ldc + n) * 2) = w;
          }
      return;
    }
  }
  finish<RAW>(p, acc, row0 + wr, col0 + wc, lane);
}

// An operand panel from stage s0 on: K-major rows start s0 * ROW bytes later, M/N-major ones s0 * BK k rows later;
// the bytes to the matrix's end shrink by as much.
template<class Sh>
__device__ __forceinline__ cairn::tile::Panel from_stage(cairn::tile::Panel pn, bool kmajor, int s0, std::int64_t ld) {
  const std::int64_t skip = kmajor ? std::int64_t(s0) * Sh::ROW : std::int64_t(s0) * Sh::BK * ld * Sh::ES;
  return cairn::tile::Panel{pn.start + skip, pn.bytes - skip};
}

// The 32-bit pattern of a value (an f32 or int32 accumulator element, taken by value: a bit cast straight from an
// element of the accumulator vector read element 0 for every element, as compiled here).
template<class T> __device__ __forceinline__ std::uint32_t bits32(T x) {
  static_assert(sizeof(T) == 4, "a 32-bit accumulator");
  return __builtin_bit_cast(std::uint32_t, x);
}

// A partial tile of the split round: the accumulators' 32-bit patterns (f32 sums, or exact int32 ones) as a BM x BN
// row-major tile at `part`, 16 bytes a quad (the fixup reads them back in the same layout).
template<class Sh, class Acc, int FM, int FN>
__device__ __forceinline__ void store_partial(const Acc (&acc)[FM][FN], void* part, int wr, int wc, int lane) {
  char* base = static_cast<char*>(part);
#pragma unroll
  for(int i = 0; i < FM; ++i)
#pragma unroll
    for(int j = 0; j < FN; ++j)
#pragma unroll
      for(int q = 0; q < 4; ++q) {
        const int m = wr + 32 * i + cairn::tile::acc_m(lane), n = wc + 32 * j + cairn::tile::acc_n(lane, q);
        u32x4 w;
#pragma unroll
        for(int e = 0; e < 4; ++e) w[e] = bits32(acc[i][j][4 * q + e]);  // the element's value, then its pattern
        *reinterpret_cast<u32x4*>(base + (std::int64_t(m) * Sh::BN + n) * 4) = w;
      }
}

// Where a tile's time goes: a Clock is told when the tile starts, when its first MFMA is about to issue (the
// prologue's loads of stage 0 have landed), when the main loop ends, when the epilogue's stores are issued and when
// they are done (mark<0> .. mark<4>; the last comes after a wait for every store), then handed the parameters and the
// tile (record). The library's kernels take NoClock, which does nothing and adds no instruction; a clock-stamp build
// (tests/cpp/wave_stamps.hip) supplies one that reads the shader and reference clocks.
struct NoClock {
  template<int POINT> __device__ __forceinline__ void mark() {}
  __device__ __forceinline__ void record(const Params&, int, int, int, int) {}
  static constexpr bool on = false;
};

// One output tile (tm, tn) over the k stages from s0 on: k counts the operands' elements from stage s0 (all of k
// for a whole tile; a segment's share in the split round). With PART the accumulators go to `part` as a partial
// tile (store_partial), else through the epilogue into c. lds is the workgroup's ring, terms its epilogue terms.
template<class Sh, int OP, bool TA, bool TB, bool RAW, bool PART, class Clock = NoClock>
__device__ __forceinline__ void wave_tile(const Params& p, char* lds, float* terms, int tm, int tn, int s0, int k,
                                          void* part) {
  static_assert(Sh::WAVES == 4, "one wave a SIMD");
  Clock clock;
  clock.template mark<0>();
  using M = Mfma<OP>;
  using Acc = typename M::Acc;
  constexpr bool AK = !TA, BKM = TB;
  constexpr int S = Sh::STAGES, FM = Sh::FM, FN = Sh::FN, ES = Sh::ES;
  constexpr int LOADS = Sh::LOADS_A + Sh::LOADS_B;  // this thread's 16-byte loads a stage
  constexpr int RA = AK ? FM : 2 * FM, RB = BKM ? FN : 2 * FN, READS = RA + RB;  // LDS reads a k-step
  static_assert(READS <= 32 && LOADS <= 8, "the interleave below places these between 16 MFMAs");

  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  int wr, wc;
  wave_origin<Sh>(wave, wr, wc);
  const int row0 = tm * Sh::BM, col0 = tn * Sh::BN;
  const Terms mine_terms = RAW || PART ? Terms{} : prefetch_terms<Sh>(p, row0, col0, t);
  const cairn::tile::Panel pa = from_stage<Sh>(cairn::tile::panel(AK, row0, p.m, p.k, p.lda, ES), AK, s0, p.lda);
  const cairn::tile::Panel pb = from_stage<Sh>(cairn::tile::panel(BKM, col0, p.n, p.k, p.ldb, ES), BKM, s0, p.ldb);
  const char* a = static_cast<const char*>(p.a) + pa.start;
  const char* b = static_cast<const char*>(p.b) + pb.start;
  const unsigned ring = lds_address(lds);

  Dma dma;
  Loader<Sh, Sh::BM, AK, Dma> la;
  Loader<Sh, Sh::BN, BKM, Dma> lb;  // the host runs this kernel only where both loaders' imm_fits holds
  la.setup(t, row0, p.m, p.lda);
  lb.setup(t, col0, p.n, p.ldb);
  const int T = (k + Sh::BK - 1) / Sh::BK;

  Acc acc[FM][FN];
#pragma unroll
  for(int i = 0; i < FM; ++i)
#pragma unroll
    for(int j = 0; j < FN; ++j) acc[i][j] = Acc{};
  u32x4 xa[2][FM], xb[2][FN];
  // The lane's transpose-read offset of each 32-column block of an M/N-major operand at k-step 0, half 0; the
  // other k-step and half add mnmajor_step, an immediate.
  int ta_off[FM], tb_off[FN];
#pragma unroll
  for(int i = 0; i < FM; ++i) ta_off[i] = AK ? 0 : mnmajor_fragment<ES, Sh::BM>(wr + 32 * i, 0, 0, lane);
#pragma unroll
  for(int j = 0; j < FN; ++j) tb_off[j] = BKM ? 0 : mnmajor_fragment<ES, Sh::BN>(wc + 32 * j, 0, 0, lane);
  // The same offsets two stages on. Ring slots 2 and 3 start 64 KiB or more into the ring, past the 16-bit offset
  // field of an LDS read; from these bases their reads keep an immediate offset, with no address add in the loop.
  // Opaque to the compiler, which would otherwise fold them back into the offsets above plus a constant too large.
  int ta_hi[FM], tb_hi[FN];
#pragma unroll
  for(int i = 0; i < FM; ++i) {
    ta_hi[i] = ta_off[i] + 2 * Sh::STAGE;
    asm volatile("" : "+v"(ta_hi[i]));
  }
#pragma unroll
  for(int j = 0; j < FN; ++j) {
    tb_hi[j] = tb_off[j] + 2 * Sh::STAGE;
    asm volatile("" : "+v"(tb_hi[j]));
  }

  // A stage's place in the ring: `slot` is its index there, a constant in the unrolled steady loop (so that every LDS
  // address and M0 value is an immediate) or an int.
  auto stage_at = [&](auto slot) { return lds + int(slot) * Sh::STAGE; };
  // Read X of a k-step's READS from ring slot `slot` (a constant in the unrolled steady loop, else an int): a's
  // fragments first (one b128 each, or two transpose halves), then b's.
  auto read = [&](auto buf, auto slot, auto s, auto x) {
    constexpr int X = decltype(x)::value, BUF = decltype(buf)::value, KS = decltype(s)::value;
    const char* stage = stage_at(slot);
    // The first byte of a transpose read's block i at k-step 0, half 0, from lo (slot's offsets) or hi.
    auto block = [&](const auto& lo, const auto& hi, int i) -> const char* {
      if constexpr(std::is_integral_v<decltype(slot)>) return stage + lo[i];
      else if constexpr(decltype(slot)::value >= 2) return lds + hi[i] + (decltype(slot)::value - 2) * Sh::STAGE;
      else return stage + lo[i];
    };
    if constexpr(X < RA) {
      if constexpr(AK) xa[BUF][X] = *reinterpret_cast<const u32x4*>(stage + kmajor_fragment(wr + 32 * X, KS, lane));
      else {
        const u32x2 h = transpose_half<ES>(block(ta_off, ta_hi, X / 2) + mnmajor_step<ES, Sh::BM>(KS, X % 2));
        xa[BUF][X / 2][2 * (X % 2)] = h[0];
        xa[BUF][X / 2][2 * (X % 2) + 1] = h[1];
      }
    } else {
      constexpr int Y = X - RA;
      const char* bs = stage + Sh::A_BYTES;
      if constexpr(BKM) xb[BUF][Y] = *reinterpret_cast<const u32x4*>(bs + kmajor_fragment(wc + 32 * Y, KS, lane));
      else {
        const u32x2 h = transpose_half<ES>(block(tb_off, tb_hi, Y / 2) + Sh::A_BYTES + mnmajor_step<ES, Sh::BN>(KS, Y % 2));
        xb[BUF][Y / 2][2 * (Y % 2)] = h[0];
        xb[BUF][Y / 2][2 * (Y % 2) + 1] = h[1];
      }
    }
  };
  auto mfma = [&](auto buf, auto x) {
    constexpr int X = decltype(x)::value, BUF = decltype(buf)::value, I = X / FN, J = X % FN;
    acc[I][J] = M::step(xb[BUF][J], xa[BUF][I], acc[I][J]);
  };
  using LA = Loader<Sh, Sh::BM, AK, Dma>;
  using LB = Loader<Sh, Sh::BN, BKM, Dma>;
  // One operand's part of stage st (ring slot `slot`): M0 once, then its loads by immediate offset; with `tail`, each
  // chunk checked against k (Loader::load_imm), else as set up (Loader::load_steady, for stages that end at or before
  // k and those past the last).
  using Tail = std::true_type;
  using Steady = std::false_type;
  auto load_a = [&](const auto& r, int st, auto slot, auto u, auto tail) {
    constexpr int U = decltype(u)::value;
    if constexpr(U == 0) dma.set_base(LA::base(ring + unsigned(int(slot) * Sh::STAGE), wave));
    if constexpr(decltype(tail)::value) la.template load_imm<U>(dma, r, st, k);
    else la.template load_steady<U>(dma, r);
  };
  auto load_b = [&](const auto& r, int st, auto slot, auto u, auto tail) {
    constexpr int U = decltype(u)::value;
    if constexpr(U == 0) dma.set_base(LB::base(ring + unsigned(int(slot) * Sh::STAGE + Sh::A_BYTES), wave));
    if constexpr(decltype(tail)::value) lb.template load_imm<U>(dma, r, st, k);
    else lb.template load_steady<U>(dma, r);
  };
  auto stage_a = [&](int st) {
    const auto r = la.resource(dma, a, pa.bytes, p.lda, st);
    unrolled<Sh::LOADS_A>([&](auto u) { load_a(r, st, st % S, u, Tail{}); });
  };
  auto stage_b = [&](int st) {
    const auto r = lb.resource(dma, b, pb.bytes, p.ldb, st);
    unrolled<Sh::LOADS_B>([&](auto u) { load_b(r, st, st % S, u, Tail{}); });
  };

  using B0 = std::integral_constant<int, 0>;
  using B1 = std::integral_constant<int, 1>;
  // Stages 0 .. S - 2 whole and a's part of stage S - 1; iteration 0 brings b's part of stage S - 1.
  for(int st = 0; st < S - 1; ++st) {
    stage_a(st);
    stage_b(st);
  }
  stage_a(S - 1);
  using K0 = std::integral_constant<int, 0>;
  using K1 = std::integral_constant<int, 1>;
  wait_loads<(S - 2) * LOADS + Sh::LOADS_A>();
  fenced_barrier();
  unrolled<READS>([&](auto x) { read(B0{}, K0{}, K0{}, x); });
  clock.template mark<1>();

  // The loop's buffer resources, walked a stage at a time: b's from stage S - 1 (iteration 0 loads its b), a's from
  // stage S. Each is computed after MFMAs 8 (its bytes) and 9 (the resource) of the k-step before the one that loads
  // it, and its walk advanced after MFMA 12: slots with no other issue.
  Walk wa = walk<Sh, AK>(a, pa.bytes, p.lda, S), wb = walk<Sh, BKM>(b, pb.bytes, p.ldb, S - 1);
  Dma::Rsrc rb = Dma::resource(wb), ra;
  unsigned records;
  wb.advance();
  // Iterations before `steady` load only stages that end at or before k, or (where k is a whole number of stages)
  // stages past the last: their loads skip the per-chunk k check. The others load the last, partial, stage.
  const int steady = k % Sh::BK == 0 ? T : (T - 1 - S > 0 ? T - 1 - S : 0);

  // Placing: reads 2 X and 2 X + 1 of a k-step after MFMA X, so that they complete well before their MFMAs; load u of
  // a half stage after MFMA 4 u + 2.
  static_assert(Sh::LOADS_A <= 4 && Sh::LOADS_B <= 4, "a half stage's loads take every fourth MFMA");
  static_assert(READS <= 16, "MFMAs 8, 9 and 12 of a k-step issue no read");
  // Iteration `it`, its stage in ring slot `slot` (= it % S; the next in slot + 1, b's loads this iteration go to
  // slot + S - 1 and a's to slot itself, all mod S).
  auto iteration = [&](int it, auto slot, auto tail) {
    const auto next = [&] {
      if constexpr(std::is_integral_v<decltype(slot)>) return (slot + 1) % S;
      else return std::integral_constant<int, (decltype(slot)::value + 1) % S>{};
    }();
    const auto slot_b = [&] {
      if constexpr(std::is_integral_v<decltype(slot)>) return (slot + S - 1) % S;
      else return std::integral_constant<int, (decltype(slot)::value + S - 1) % S>{};
    }();
    const int sb = it + S - 1, sa = it + S;  // the stages whose b's, then a's, loads this iteration issues
    unrolled<16>([&](auto x) {
      constexpr int X = decltype(x)::value;
      mfma(B0{}, x);
      fence();
      if constexpr(2 * X < READS) read(B1{}, slot, K1{}, std::integral_constant<int, 2 * X>{});
      if constexpr(2 * X + 1 < READS) read(B1{}, slot, K1{}, std::integral_constant<int, 2 * X + 1>{});
      if constexpr(X % 4 == 2 && X / 4 < Sh::LOADS_B) load_b(rb, sb, slot_b, std::integral_constant<int, X / 4>{}, tail);
      if constexpr(X == 8) records = wa.records();
      if constexpr(X == 9) ra = Dma::resource(wa.at, records);
      if constexpr(X == 12) {
        wa.advance();
        pin(wa);
      }
      fence();
    });
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    wait_loads<(S - 2) * LOADS>();
    fenced_barrier();
    unrolled<16>([&](auto x) {
      constexpr int X = decltype(x)::value;
      mfma(B1{}, x);
      fence();
      if constexpr(2 * X < READS) read(B0{}, next, K0{}, std::integral_constant<int, 2 * X>{});
      if constexpr(2 * X + 1 < READS) read(B0{}, next, K0{}, std::integral_constant<int, 2 * X + 1>{});
      if constexpr(X % 4 == 2 && X / 4 < Sh::LOADS_A) load_a(ra, sa, slot, std::integral_constant<int, X / 4>{}, tail);
      if constexpr(X == 8) records = wb.records();
      if constexpr(X == 9) rb = Dma::resource(wb.at, records);
      if constexpr(X == 12) {
        wb.advance();
        pin(wb);
      }
      fence();
    });
  };
  // The steady iterations S at a time, each of the S with its ring slot known; then the rest one at a time.
  int it = 0;
  for(; it + S <= steady; it += S)
    unrolled<S>([&](auto u) { iteration(it + decltype(u)::value, u, Steady{}); });
  for(; it < T; ++it) iteration(it, it % S, Tail{});
  clock.template mark<2>();
  wait_loads<0>();  // the loads past the last stage land before the workgroup's LDS is given back

  if constexpr(PART) store_partial<Sh>(acc, part, wr, wc, lane);
  else store_tile<Sh, RAW>(p, acc, lds, terms, mine_terms, wave, row0, col0, wr, wc, lane);
  if constexpr(Clock::on) {
    clock.template mark<3>();
    wait_loads<0>();
    clock.template mark<4>();
    clock.record(p, tm, tn, wave, lane);
  }
}

// The ring and the epilogue terms (3 KiB: past the staged store's part of the ring where the ring has room, a
// 5-stage ring, else an array of their own), declared by each kernel.
#define CAIRN_WAVE_LDS(Sh)                                                                                          \
  __shared__ __attribute__((aligned(1024))) char lds[Sh::STAGES * Sh::STAGE];                                     \
  float* terms;                                                                                                   \
  if constexpr(Sh::STAGES * Sh::STAGE >= Sh::WTM * 256 * Sh::WAVES + 3 * 1024)                                   \
    terms = reinterpret_cast<float*>(lds + Sh::WTM * 256 * Sh::WAVES);                                            \
  else {                                                                                                          \
    __shared__ float own[3 * 256];                                                                                \
    terms = own;                                                                                                  \
  }

// The whole-tile pass: workgroup b runs the tile of id whole_id(b) over all of k.
template<class Sh, int OP, bool TA, bool TB, bool RAW>
__global__ void __launch_bounds__(256) wave_gemm(Params p) {
  CAIRN_WAVE_LDS(Sh)
  int tm, tn;
  cairn::tile::tile_at(cairn::tile::whole_id(p.split, int(blockIdx.x)), p.tiles_m, p.tiles_n, p.group, tm, tn);
  wave_tile<Sh, OP, TA, TB, RAW, false>(p, lds, terms, tm, tn, 0, p.k, nullptr);
}

// The split round: workgroup u, unit u / xcds of XCD u % xcds, runs its one or two segments (split_segment) into
// its partial slots 2 u and 2 u + 1.
template<class Sh, int OP, bool TA, bool TB>
__global__ void __launch_bounds__(256) wave_split(Params p) {
  CAIRN_WAVE_LDS(Sh)
  const int u = int(blockIdx.x), x = u % p.split.xcds, v = u / p.split.xcds;  // unit v of XCD x
  for(int j = 0; j < 2; ++j) {
    int tile, s0, s1;
    if(!cairn::tile::split_segment(p.split, v, j, tile, s0, s1)) break;  // the same for every thread
    if(j) {  // every wave is past its LDS reads of the first segment before the second refills the ring
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      fenced_barrier();
    }
    int tm, tn;
    cairn::tile::tile_at(cairn::tile::split_id(p.split, x, tile), p.tiles_m, p.tiles_n, p.group, tm, tn);
    const int k = (p.k < s1 * Sh::BK ? p.k : s1 * Sh::BK) - s0 * Sh::BK;
    void* slot = static_cast<char*>(p.work) + std::int64_t(2 * u + j) * (Sh::BM * Sh::BN * 4);
    wave_tile<Sh, OP, TA, TB, false, true>(p, lds, terms, tm, tn, s0, k, slot);
  }
}

// The 8-bit floats on the same ring: one v_mfma_f32_32x32x64_f8f6f4 covers a whole stage (64 bytes of k), so a
// stage's fragments, both 16-byte k-steps of the int8 layout, are read during the previous stage's MFMAs, double-
// buffered by stage. Iteration `it`:
//   wait for this wave's loads of stage it + 1 and its own LDS reads; barrier;
//   the 16 MFMAs of stage it, between them the fragment reads of stage it + 1 and the loads of stage it + STAGES
//   into the buffer stage it used (every wave has stage it in registers once past the barrier).
// The hazards are the ones of wave_gemm, ordered by the one barrier a stage.
template<class Sh, int OP, bool TA, bool TB, bool PART>
__device__ __forceinline__ void wave8_tile(const Params& p, char* lds, float* terms, int tm, int tn, int s0, int k,
                                           void* part) {
  static_assert(Sh::WAVES == 4 && Sh::ES == 1, "one wave a SIMD, 8-bit operands");
  using M = Mfma<OP>;
  using Acc = typename M::Acc;
  constexpr bool AK = !TA, BKM = TB;
  constexpr int S = Sh::STAGES, FM = Sh::FM, FN = Sh::FN, ES = Sh::ES;
  constexpr int LOADS = Sh::LOADS_A + Sh::LOADS_B;
  constexpr int RA = AK ? FM : 2 * FM, RB = BKM ? FN : 2 * FN, STEP_READS = RA + RB, READS = 2 * STEP_READS;
  static_assert(READS <= 32 && Sh::LOADS_A <= 4 && Sh::LOADS_B <= 4, "the interleave below");

  const int t = threadIdx.x, lane = t & 63;
  const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
  int wr, wc;
  wave_origin<Sh>(wave, wr, wc);
  const int row0 = tm * Sh::BM, col0 = tn * Sh::BN;
  const Terms mine_terms = PART ? Terms{} : prefetch_terms<Sh>(p, row0, col0, t);
  const cairn::tile::Panel pa = from_stage<Sh>(cairn::tile::panel(AK, row0, p.m, p.k, p.lda, ES), AK, s0, p.lda);
  const cairn::tile::Panel pb = from_stage<Sh>(cairn::tile::panel(BKM, col0, p.n, p.k, p.ldb, ES), BKM, s0, p.ldb);
  const char* a = static_cast<const char*>(p.a) + pa.start;
  const char* b = static_cast<const char*>(p.b) + pb.start;
  const unsigned ring = lds_address(lds);

  Dma dma;
  Loader<Sh, Sh::BM, AK, Dma> la;
  Loader<Sh, Sh::BN, BKM, Dma> lb;  // the host runs this kernel only where both loaders' imm_fits holds
  la.setup(t, row0, p.m, p.lda);
  lb.setup(t, col0, p.n, p.ldb);
  const int T = (k + Sh::BK - 1) / Sh::BK;
  using LA = Loader<Sh, Sh::BM, AK, Dma>;
  using LB = Loader<Sh, Sh::BN, BKM, Dma>;
  // A stage's place in the ring (a constant in the unrolled steady loop, else an int), and one operand's part of stage
  // st there: M0 once, then its loads by immediate offset, each chunk checked against k only with `tail`.
  using Tail = std::true_type;
  using Steady = std::false_type;
  auto stage_at = [&](auto slot) { return lds + int(slot) * Sh::STAGE; };
  auto load_a = [&](const auto& r, int st, auto slot, auto u, auto tail) {
    constexpr int U = decltype(u)::value;
    if constexpr(U == 0) dma.set_base(LA::base(ring + unsigned(int(slot) * Sh::STAGE), wave));
    if constexpr(decltype(tail)::value) la.template load_imm<U>(dma, r, st, k);
    else la.template load_steady<U>(dma, r);
  };
  auto load_b = [&](const auto& r, int st, auto slot, auto u, auto tail) {
    constexpr int U = decltype(u)::value;
    if constexpr(U == 0) dma.set_base(LB::base(ring + unsigned(int(slot) * Sh::STAGE + Sh::A_BYTES), wave));
    if constexpr(decltype(tail)::value) lb.template load_imm<U>(dma, r, st, k);
    else lb.template load_steady<U>(dma, r);
  };
  auto stage_all = [&](int st) {
    const auto ra = la.resource(dma, a, pa.bytes, p.lda, st);
    unrolled<Sh::LOADS_A>([&](auto u) { load_a(ra, st, st % S, u, Tail{}); });
    const auto rb = lb.resource(dma, b, pb.bytes, p.ldb, st);
    unrolled<Sh::LOADS_B>([&](auto u) { load_b(rb, st, st % S, u, Tail{}); });
  };

  Acc acc[FM][FN];
#pragma unroll
  for(int i = 0; i < FM; ++i)
#pragma unroll
    for(int j = 0; j < FN; ++j) acc[i][j] = Acc{};
  u32x4 xa[2][2][FM], xb[2][2][FN];  // [buffer][k-step of the stage][block]
  int ta_off[FM], tb_off[FN];        // transpose-read offsets at k-step 0, half 0 (mnmajor_step adds the rest)
#pragma unroll
  for(int i = 0; i < FM; ++i) ta_off[i] = AK ? 0 : mnmajor_fragment<ES, Sh::BM>(wr + 32 * i, 0, 0, lane);
#pragma unroll
  for(int j = 0; j < FN; ++j) tb_off[j] = BKM ? 0 : mnmajor_fragment<ES, Sh::BN>(wc + 32 * j, 0, 0, lane);
  int ta_hi[FM], tb_hi[FN];  // the same two stages on, opaque: ring slots 2 and 3 (as in wave_gemm)
#pragma unroll
  for(int i = 0; i < FM; ++i) {
    ta_hi[i] = ta_off[i] + 2 * Sh::STAGE;
    asm volatile("" : "+v"(ta_hi[i]));
  }
#pragma unroll
  for(int j = 0; j < FN; ++j) {
    tb_hi[j] = tb_off[j] + 2 * Sh::STAGE;
    asm volatile("" : "+v"(tb_hi[j]));
  }
  // Read X of a stage's READS from ring slot `slot`: k-step X / STEP_READS, then as wave_gemm orders a k-step's reads.
  auto read = [&](auto buf, auto slot, auto x) {
    constexpr int BUF = decltype(buf)::value, X = decltype(x)::value % STEP_READS, s = decltype(x)::value / STEP_READS;
    const char* stage = stage_at(slot);
    auto block = [&](const auto& lo, const auto& hi, int i) -> const char* {
      if constexpr(std::is_integral_v<decltype(slot)>) return stage + lo[i];
      else if constexpr(decltype(slot)::value >= 2) return lds + hi[i] + (decltype(slot)::value - 2) * Sh::STAGE;
      else return stage + lo[i];
    };
    if constexpr(X < RA) {
      if constexpr(AK) xa[BUF][s][X] = *reinterpret_cast<const u32x4*>(stage + kmajor_fragment(wr + 32 * X, s, lane));
      else {
        const u32x2 h = transpose_half<ES>(block(ta_off, ta_hi, X / 2) + mnmajor_step<ES, Sh::BM>(s, X % 2));
        xa[BUF][s][X / 2][2 * (X % 2)] = h[0];
        xa[BUF][s][X / 2][2 * (X % 2) + 1] = h[1];
      }
    } else {
      constexpr int Y = X - RA;
      const char* bs = stage + Sh::A_BYTES;
      if constexpr(BKM) xb[BUF][s][Y] = *reinterpret_cast<const u32x4*>(bs + kmajor_fragment(wc + 32 * Y, s, lane));
      else {
        const u32x2 h = transpose_half<ES>(block(tb_off, tb_hi, Y / 2) + Sh::A_BYTES + mnmajor_step<ES, Sh::BN>(s, Y % 2));
        xb[BUF][s][Y / 2][2 * (Y % 2)] = h[0];
        xb[BUF][s][Y / 2][2 * (Y % 2) + 1] = h[1];
      }
    }
  };
  auto mfma = [&](auto buf, auto x) {
    constexpr int BUF = decltype(buf)::value, I = decltype(x)::value / FN, J = decltype(x)::value % FN;
    acc[I][J] = M::step(xb[BUF][0][J], xb[BUF][1][J], xa[BUF][0][I], xa[BUF][1][I], acc[I][J]);
  };
  // Stages 0 .. S - 1 (every buffer starts free), then stage 0's fragments.
  for(int st = 0; st < S; ++st) stage_all(st);
  wait_loads<(S - 1) * LOADS>();
  fenced_barrier();
  unrolled<READS>([&](auto x) { read(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{}, x); });

  // Iteration `it` loads stage it + S into the slot stage it leaves. Its resources are walked a stage at a time and
  // made after MFMAs 12 .. 15 of the iteration before, slots no load uses; steady iterations (stages that end
  // at or before k, or past the last where k is whole stages) skip the per-chunk k check.
  Walk wa = walk<Sh, AK>(a, pa.bytes, p.lda, S), wb = walk<Sh, BKM>(b, pb.bytes, p.ldb, S);
  Dma::Rsrc ra = Dma::resource(wa), rb = Dma::resource(wb);
  wa.advance();
  wb.advance();
  unsigned records;
  const int steady = k % Sh::BK == 0 ? T : (T - 1 - S > 0 ? T - 1 - S : 0);
  // A 32x32x64 fp8 MFMA takes 64 cycles: between two, fifteen issue slots, room for two reads and the walk's work.
  static_assert(8 + Sh::LOADS_B <= 12, "MFMAs 12 .. 15 of a stage issue no load");
  auto iteration = [&](int it, auto slot, auto cur, auto tail) {
    constexpr int C = decltype(cur)::value, N = 1 - C;
    const auto next = [&] {
      if constexpr(std::is_integral_v<decltype(slot)>) return (slot + 1) % S;
      else return std::integral_constant<int, (decltype(slot)::value + 1) % S>{};
    }();
    const int sl = it + S;  // the stage whose loads this iteration issues, into stage it's slot
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    wait_loads<(S - 2) * LOADS>();
    fenced_barrier();
    unrolled<FM * FN>([&](auto x) {
      constexpr int X = decltype(x)::value;
      mfma(std::integral_constant<int, C>{}, x);
      fence();
      if constexpr(2 * X < READS) read(std::integral_constant<int, N>{}, next, std::integral_constant<int, 2 * X>{});
      if constexpr(2 * X + 1 < READS) read(std::integral_constant<int, N>{}, next, std::integral_constant<int, 2 * X + 1>{});
      if constexpr(X >= 4 && X < 4 + Sh::LOADS_A) load_a(ra, sl, slot, std::integral_constant<int, X - 4>{}, tail);
      if constexpr(X >= 8 && X < 8 + Sh::LOADS_B) load_b(rb, sl, slot, std::integral_constant<int, X - 8>{}, tail);
      if constexpr(X == 12) records = wa.records();
      if constexpr(X == 13) {
        ra = Dma::resource(wa.at, records);
        wa.advance();
        pin(wa);
      }
      if constexpr(X == 14) records = wb.records();
      if constexpr(X == 15) {
        rb = Dma::resource(wb.at, records);
        wb.advance();
        pin(wb);
      }
      fence();
    });
  };
  // Steady iterations S at a time (S is even, so each one's register buffer and ring slot are constants), then the
  // rest one at a time.
  static_assert(S % 2 == 0, "the register buffers alternate within an unrolled group");
  int it = 0;
  for(; it + S <= steady; it += S)
    unrolled<S>([&](auto u) { iteration(it + decltype(u)::value, u, std::integral_constant<int, decltype(u)::value % 2>{}, Steady{}); });
  for(; it < T; ++it) {
    if(it & 1) iteration(it, it % S, std::integral_constant<int, 1>{}, Tail{});
    else iteration(it, it % S, std::integral_constant<int, 0>{}, Tail{});
  }
  wait_loads<0>();  // the loads past the last stage land before the workgroup's LDS is given back
  if constexpr(PART) store_partial<Sh>(acc, part, wr, wc, lane);
  else store_tile<Sh, false>(p, acc, lds, terms, mine_terms, wave, row0, col0, wr, wc, lane);
}

template<class Sh, int OP, bool TA, bool TB>
__global__ void __launch_bounds__(256) wave8_gemm(Params p) {
  CAIRN_WAVE_LDS(Sh)
  int tm, tn;
  cairn::tile::tile_at(cairn::tile::whole_id(p.split, int(blockIdx.x)), p.tiles_m, p.tiles_n, p.group, tm, tn);
  wave8_tile<Sh, OP, TA, TB, false>(p, lds, terms, tm, tn, 0, p.k, nullptr);
}

template<class Sh, int OP, bool TA, bool TB>
__global__ void __launch_bounds__(256) wave8_split(Params p) {
  CAIRN_WAVE_LDS(Sh)
  const int u = int(blockIdx.x), x = u % p.split.xcds, v = u / p.split.xcds;
  for(int j = 0; j < 2; ++j) {
    int tile, s0, s1;
    if(!cairn::tile::split_segment(p.split, v, j, tile, s0, s1)) break;
    if(j) {
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      fenced_barrier();
    }
    int tm, tn;
    cairn::tile::tile_at(cairn::tile::split_id(p.split, x, tile), p.tiles_m, p.tiles_n, p.group, tm, tn);
    const int k = (p.k < s1 * Sh::BK ? p.k : s1 * Sh::BK) - s0 * Sh::BK;
    void* slot = static_cast<char*>(p.work) + std::int64_t(2 * u + j) * (Sh::BM * Sh::BN * 4);
    wave8_tile<Sh, OP, TA, TB, true>(p, lds, terms, tm, tn, s0, k, slot);
  }
}

// The split round's fixup: block (f, r), split tile f / xcds of XCD f % xcds (so that it runs on that XCD, whose L2
// holds the partials its units wrote), rows 4 r .. 4 r + 3; thread th one quad (4 columns) of row 4 r + th / 64. It
// adds the tile's partials in the order of their units (their k order), then applies the epilogue's steps and stores
// c as the whole-tile pass would. INT: the partials are exact int32 sums (int8 operands), added as integers.
template<int BM, int BN, bool INT>
__global__ void __launch_bounds__(256) split_fixup(Params p) {
  static_assert(BN == 256, "64 quads a row");
  const int f = int(blockIdx.x), x = f % p.split.xcds, t = f / p.split.xcds;
  const int row_in = 4 * int(blockIdx.y) + int(threadIdx.x) / 64, col_in = 4 * (int(threadIdx.x) % 64);
  int tm, tn;
  cairn::tile::tile_at(cairn::tile::split_id(p.split, x, t), p.tiles_m, p.tiles_n, p.group, tm, tn);
  const int m = tm * BM + row_in, n = tn * BN + col_in;
  if(m >= p.m || n >= p.n) return;  // n and p.n are multiples of 4: a quad is in or out whole
  int first, last;
  cairn::tile::split_units_of(p.split, t, first, last);
  const std::int64_t within = (std::int64_t(row_in) * BN + col_in) * 4;
  u32x4 sum = *reinterpret_cast<const u32x4*>(static_cast<const char*>(p.work) +
                                             std::int64_t(cairn::tile::split_slot(p.split, x, t, first)) * (BM * BN * 4) + within);
  for(int v = first + 1; v <= last; ++v) {
    const u32x4 w = *reinterpret_cast<const u32x4*>(static_cast<const char*>(p.work) +
                                                   std::int64_t(cairn::tile::split_slot(p.split, x, t, v)) * (BM * BN * 4) + within);
#pragma unroll
    for(int e = 0; e < 4; ++e) {
      if constexpr(INT) sum[e] = std::uint32_t(int(sum[e]) + int(w[e]));
      else sum[e] = as_bits(from_bits(sum[e]) + from_bits(w[e]));
    }
  }
  char* c = static_cast<char*>(p.c);
  const std::int64_t at = std::int64_t(m) * p.ldc + n;
  if(INT && p.c_type == CAIRN_TYPE_I32) {
    *reinterpret_cast<u32x4*>(c + at * 4) = sum;
    return;
  }
  with_form(p, [&](auto form) {
    using F = decltype(form);
    const float rs = p.row_scale ? p.row_scale[m] : 1.0f;
    float v[4];
#pragma unroll
    for(int e = 0; e < 4; ++e) {
      const float acc = INT ? float(int(sum[e])) : from_bits(sum[e]);
      const float cs = p.col_scale ? p.col_scale[n + e] : 1.0f;
      const float bs = !p.bias ? -0.0f
                       : p.bias_type == CAIRN_TYPE_BF16 ? widen_bf16(static_cast<const std::uint16_t*>(p.bias)[n + e])
                                                        : static_cast<const float*>(p.bias)[n + e];
      v[e] = apply<F>(acc, rs, cs, bs);
    }
    if(p.c_type == CAIRN_TYPE_F32) {
      float* out = reinterpret_cast<float*>(c + at * 4);
      if(p.accumulate)
#pragma unroll
        for(int e = 0; e < 4; ++e) v[e] = out[e] + v[e];
      *reinterpret_cast<float4*>(out) = float4{v[0], v[1], v[2], v[3]};
    } else if(p.c_type == CAIRN_TYPE_BF16) {
      *reinterpret_cast<u32x2*>(c + at * 2) = u32x2{narrow2_bf16(v[0], v[1]), narrow2_bf16(v[2], v[3])};
    } else {
      *reinterpret_cast<u32x2*>(c + at * 2) =
          u32x2{std::uint32_t(narrow_f16(v[0])) | (std::uint32_t(narrow_f16(v[1])) << 16),
                std::uint32_t(narrow_f16(v[2])) | (std::uint32_t(narrow_f16(v[3])) << 16)};
    }
  });
}

// A launch: the whole-tile pass (whole_tiles workgroups), then, where the last round is split, the split pass and its
// fixup, all on the stream in order.
template<class Sh, bool INT> hipError_t launch_fixup(const Params& p, hipStream_t s) {
  hipLaunchKernelGGL((split_fixup<Sh::BM, Sh::BN, INT>), dim3(unsigned(p.split.xcds * p.split.tiles), unsigned(Sh::BM / 4)),
                     dim3(256), 0, s, p);
  return hipGetLastError();
}

template<class Sh, int OP, bool TA, bool TB> hipError_t launch_wave8(const Params& p, hipStream_t s) {
  if(p.whole_tiles) hipLaunchKernelGGL((wave8_gemm<Sh, OP, TA, TB>), dim3(unsigned(p.whole_tiles)), dim3(256), 0, s, p);
  if(p.split.tiles) {
    hipLaunchKernelGGL((wave8_split<Sh, OP, TA, TB>), dim3(unsigned(p.split.xcds * p.split.units)), dim3(256), 0, s, p);
    if(const hipError_t e = hipGetLastError(); e != hipSuccess) return e;
    return launch_fixup<Sh, false>(p, s);
  }
  return hipGetLastError();
}

template<class Sh, int OP, bool TA, bool TB> hipError_t launch_wave(const Params& p, hipStream_t s) {
  constexpr bool INT = OP == OP_I8;
  if(p.whole_tiles) {
    if(INT && p.c_type == CAIRN_TYPE_I32)
      hipLaunchKernelGGL((wave_gemm<Sh, OP, TA, TB, INT>), dim3(unsigned(p.whole_tiles)), dim3(256), 0, s, p);
    else hipLaunchKernelGGL((wave_gemm<Sh, OP, TA, TB, false>), dim3(unsigned(p.whole_tiles)), dim3(256), 0, s, p);
  }
  if(p.split.tiles) {
    hipLaunchKernelGGL((wave_split<Sh, OP, TA, TB>), dim3(unsigned(p.split.xcds * p.split.units)), dim3(256), 0, s, p);
    if(const hipError_t e = hipGetLastError(); e != hipSuccess) return e;
    return launch_fixup<Sh, INT>(p, s);
  }
  return hipGetLastError();
}

}  // namespace cairn::gemm

// An instance of the kernel table: a launcher named NAME for one shape, operation and layout.
#define CAIRN_WAVE_INSTANCE(NAME, BM, BN, STAGES, OP, TA, TB)                                                      \
  hipError_t NAME(const cairn::gemm::Params& p, hipStream_t s) {                                                 \
    return cairn::gemm::launch_wave<                                                                              \
        cairn::pipe::Shape<BM, BN, (OP == cairn::gemm::OP_I8 ? 1 : 2), STAGES, 4>, OP, TA, TB>(p, s);           \
  }
#define CAIRN_WAVE8_INSTANCE(NAME, BM, BN, STAGES, OP, TA, TB)                                                     \
  hipError_t NAME(const cairn::gemm::Params& p, hipStream_t s) {                                                 \
    return cairn::gemm::launch_wave8<cairn::pipe::Shape<BM, BN, 1, STAGES, 4>, OP, TA, TB>(p, s);                \
  }
