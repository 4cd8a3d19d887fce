// The index arithmetic of the LDS-ring gfx950 GEMM (wave.hpp), written once for the kernel and for the host simulator
// (tests/sim/tile_sim.cpp). The simulator also runs it for eight waves a workgroup, the form of an earlier kernel.
//
// A workgroup computes a BM x BN tile. Operand tiles cross from global memory straight into LDS
// (buffer_load_dwordx4 ... lds: lane l of a wave's load writes 16 bytes at the wave's LDS base + 16 l), STAGES deep,
// 64 bytes of every row's k per stage (32 bf16/f16 or 64 int8: two MFMA k-steps). Each operand keeps the layout it
// has in memory:
//
//  - K-major (a of NN/NT, b of NT/TT): R rows of 64 bytes, chunk c of row r at physical chunk c ^ ((r >> 2) & 3);
//    an MFMA operand is one ds_read_b128 per lane.
//  - M/N-major (b of NN, a of TN/TT): k rows of R elements, chunk c of k row kk at physical chunk c ^ swz(kk):
//    4 (kk & 3) for 16-bit elements, 2 (kk & 7) for bytes (2 ((kk >> 1) & 3) where a row is only 128 bytes); an
//    MFMA operand is two LDS transpose reads per lane (ds_read_b64_tr_b16 / tr_b8), which hand each lane one column
//    of a 4 x 16 (16-bit) or 8 x 16 (byte) block that 16 lanes read row-wise.
//
// gfx950's LDS serves 64 banks of 4 bytes a clock: a ds_read_b128 in phases of 16 lanes, a 64-bit (transpose) read in
// phases of 32. The swizzles give every phase distinct banks: the 16 rows a b128 phase reads at one chunk fall on the
// four 64-byte quarters of a bank row and four chunk positions in each; the two 16-lane groups of a transpose phase
// read 4 (8) rows by 32 (16) adjacent bytes each, spread over the 16 chunk positions of a bank row. Measured as zero
// bank-conflict cycles (SQ_LDS_BANK_CONFLICT). Both operand kinds give lane l the same k for the same register
// byte: lane l holds
// k = 32 s + 16 (l / 32) + (byte of its 16), in bytes, for MFMA k-step s of the stage. So the pairing of a and b
// along k never depends on the layouts.
#pragma once
#include <cstdint>
#include "tile.hpp"

namespace cairn::pipe {
using cairn::tile::u32x4;

// WAVES 8: two groups of four waves (the earlier ping-pong form, simulated only), a wave holding (BM/2) x (BN/4)
// outputs; WAVES 4: one wave a SIMD (wave.hpp), a wave holding (BM/2) x (BN/2). Either way a stage's loads are spread over 256 threads: one
// group's for one operand (8 waves), or all four waves' for both (4 waves).
template<int BM_, int BN_, int ES_, int STAGES_, int WAVES_ = 8> struct Shape {
  static constexpr int BM = BM_, BN = BN_, ES = ES_, STAGES = STAGES_, WAVES = WAVES_;
  static constexpr int ROW = 64;             // bytes of k per operand row per stage
  static constexpr int BK = ROW / ES;        // k elements per stage: 32 or 64
  static constexpr int CE = 16 / ES;         // k elements per 16-byte chunk of a K-major row
  static constexpr int THREADS = 64 * WAVES, GROUP = 256;
  static constexpr int WTM = BM / 2, WTN = WAVES == 8 ? BN / 4 : BN / 2;  // a wave's outputs
  static constexpr int FM = WTM / 32, FN = WTN / 32;
  static constexpr int STEPS = 2;            // MFMA k-steps per stage
  static constexpr int A_BYTES = BM * ROW, B_BYTES = BN * ROW, STAGE = A_BYTES + B_BYTES;
  static constexpr int LOADS_A = BM * 4 / GROUP, LOADS_B = BN * 4 / GROUP;  // 16-byte loads per thread per stage
  static_assert(WAVES == 8 || WAVES == 4, "two groups of four waves, or one wave a SIMD");
  static_assert(BM % 64 == 0 && BN % (WAVES == 8 ? 128 : 64) == 0, "whole 32 x 32 blocks for every wave");
  static_assert(STAGES >= 3 && STAGES * STAGE <= 160 * 1024, "the ring fits the CU's LDS");
};

// The tile row and column where wave `wave`'s (WTM x WTN) block of accumulators starts: eight waves, group wave / 4
// over rows and wave % 4 over columns; four waves, a 2 x 2 grid.
template<class Sh> CAIRN_HD void wave_origin(int wave, int& r, int& c) {
  if constexpr(Sh::WAVES == 8) {
    r = (wave >> 2) * Sh::WTM;
    c = (wave & 3) * Sh::WTN;
  } else {
    r = (wave >> 1) * Sh::WTM;
    c = (wave & 1) * Sh::WTN;
  }
}

// The 16-byte LDS slot load u (of LOADS) of thread t (0..255 within its loading group) writes: 16 q bytes into the
// operand's stage, q = (LOADS wave + u) * 64 + lane. A wave's loads of one operand's stage fill LOADS consecutive KiB,
// so that one LDS base (M0) serves them all, the load's immediate offset choosing its KiB.
template<int LOADS> CAIRN_HD int slot(int t, int u) { return ((t >> 6) * LOADS + u) * 64 + (t & 63); }

// K-major: byte of (row r, chunk c), and the (row, chunk) slot q holds.
CAIRN_HD int kmajor_at(int r, int c) { return r * 64 + 16 * (c ^ ((r >> 2) & 3)); }
CAIRN_HD void kmajor_slot(int q, int& r, int& c) {
  r = q >> 2;
  c = (q & 3) ^ ((r >> 2) & 3);
}

// M/N-major with R elements a k row: byte of (k row kk, chunk c), and the (k row, chunk) slot q holds.
template<int ES, int R> CAIRN_HD int swz(int kk) {
  static_assert(R * ES >= 128, "an M/N-major k row is at least 128 bytes");
  if constexpr(ES == 2) return 4 * (kk & 3);
  else if constexpr(R >= 256) return 2 * (kk & 7);
  else return 2 * ((kk >> 1) & 3);
}
template<int ES, int R> CAIRN_HD int mnmajor_at(int kk, int c) { return kk * R * ES + 16 * (c ^ swz<ES, R>(kk)); }
template<int ES, int R> CAIRN_HD void mnmajor_slot(int q, int& kk, int& c) {
  constexpr int per = R * ES / 16;  // chunks a k row
  kk = q / per;
  c = (q % per) ^ swz<ES, R>(kk);
}

// The MFMA operand of lane l for the 32-row block at `row0`, k-step s: K-major, one 16-byte read.
CAIRN_HD int kmajor_fragment(int row0, int s, int l) { return kmajor_at(row0 + (l & 31), 2 * s + (l >> 5)); }

// M/N-major, read h of two: lane l's address for the block of columns n0 .. n0 + 31, k-step s. A 16-lane group reads
// a block of 4 (16-bit) or 8 (byte) k rows by 16 columns, row-wise; the lane then holds its column.
template<int ES, int R> CAIRN_HD int mnmajor_fragment(int n0, int s, int h, int l) {
  const int q = l & 15;
  const int cols = n0 + 16 * ((l >> 4) & 1);
  if constexpr(ES == 2) {
    const int kk = 16 * s + 8 * (l >> 5) + 4 * h + (q >> 2);
    const int col = cols + 4 * (q & 3);
    return mnmajor_at<ES, R>(kk, col >> 3) + 2 * (col & 7);
  } else {
    const int kk = 32 * s + 16 * (l >> 5) + 8 * h + (q >> 1);
    const int col = cols + 8 * (q & 1);
    return mnmajor_at<ES, R>(kk, col >> 4) + (col & 15);
  }
}

// One operand's share of a stage's loads, issued by the 256 threads of one group: R rows (a: BM, b: BN) starting at
// `first` of `total`, K-major or not. Mem supplies the buffer resource (loads past it read zero) and the 16-byte
// load into LDS: Mem::resource(const char*, int64) -> Rsrc, Mem::load_lds(Rsrc, char* wave_base, int offset).
template<class Sh, int R, bool KMAJOR, class Mem> struct Loader {
  static constexpr int LOADS = R * 4 / Sh::GROUP;
  int offset[LOADS];  // byte offset in the panel at stage 0, or OUTSIDE
  int kidx[LOADS];    // the k element (K-major: first of the chunk; else the k row) the slot holds at stage 0
  CAIRN_HD void setup(int gt, int first, int total, std::int64_t ld) {
#pragma unroll
    for(int u = 0; u < LOADS; ++u) {
      const int q = slot<LOADS>(gt, u);
      int r, c;
      if constexpr(KMAJOR) {
        kmajor_slot(q, r, c);
        offset[u] = first + r < total ? int(r * ld * Sh::ES) + 16 * c : cairn::tile::OUTSIDE;
        kidx[u] = c * Sh::CE;
      } else {
        mnmajor_slot<Sh::ES, R>(q, r, c);  // r: k row, c: chunk of 16 bytes of columns
        offset[u] = first + c * (16 / Sh::ES) < total ? int(r * ld * Sh::ES) + 16 * c : cairn::tile::OUTSIDE;
        kidx[u] = r;
      }
    }
  }
  // The buffer resource of stage `st`: the panel from the stage's first k on.
  CAIRN_HD auto resource(Mem& mem, const char* panel, std::int64_t bytes, std::int64_t ld, int st) const {
    const std::int64_t step = KMAJOR ? std::int64_t(st) * Sh::ROW : std::int64_t(st) * Sh::BK * ld * Sh::ES;
    return mem.resource(panel + step, bytes - step);
  }
  // Load u of stage `st` (resource r) into LDS at `dst` (this operand's part of the stage: a char* or an LDS
  // address), wave w's share; past k it reads zeros.
  template<class Rsrc, class Dst>
  CAIRN_HD void load_one(Mem& mem, const Rsrc& r, Dst dst, int st, int k, int u, int w) const {
    const int k0 = st * Sh::BK;
    const bool tail = k0 + Sh::BK > k;
    const int o = tail && k0 + kidx[u] >= k ? cairn::tile::OUTSIDE : offset[u];
    mem.load_lds(r, dst + (LOADS * w + u) * 1024, o);
  }
  // The same load with the wave's LDS base for this operand's stage (its first KiB, base()) already set: the load's
  // immediate offset 1024 U picks its KiB, and the lane's global offset is lowered by as much, which stays at or above
  // zero where imm_fits holds.
  template<int U, class Rsrc> CAIRN_HD void load_imm(Mem& mem, const Rsrc& r, int st, int k) const {
    const int k0 = st * Sh::BK;
    const bool tail = k0 + Sh::BK > k;
    const int o = tail && k0 + kidx[U] >= k ? cairn::tile::OUTSIDE : offset[U];
    mem.template load_lds_imm<U>(r, o);
  }
  // load_imm for a stage that ends at or before k: no chunk of it reaches past k, so the lane's offset stands as set
  // up. The main loop also issues it for stages past the last, which no MFMA reads: their bytes are never used, and
  // the walked resource (Walk) keeps every load inside the panel.
  template<int U, class Rsrc> CAIRN_HD void load_steady(Mem& mem, const Rsrc& r) const {
    mem.template load_lds_imm<U>(r, offset[U]);
  }
  template<class Dst> CAIRN_HD static Dst base(Dst dst, int w) { return dst + LOADS * w * 1024; }
  // Whether every lane's offset of load u stays at or above 1024 u for leading dimension ld: the smallest offset of
  // load u is (wave 0, lane 0) slot 64 u, row 16 u of a K-major operand (64-byte rows a stage), k row
  // 1024 u / (R ES) of an M/N-major one.
  CAIRN_HD static bool imm_fits(std::int64_t ld) { return KMAJOR ? ld * Sh::ES >= Sh::ROW : ld >= R; }
  // Stage `st` of k into LDS at `dst` (this operand's part of the ring buffer).
  template<class Dst>
  CAIRN_HD void issue(Mem& mem, const char* panel, std::int64_t bytes, std::int64_t ld, int st, int k, Dst dst, int w) {
    const auto r = resource(mem, panel, bytes, ld, st);
#pragma unroll
    for(int u = 0; u < LOADS; ++u) load_one(mem, r, dst, st, k, u, w);
  }
};

// An operand's buffer resource walked one stage at a time, as the main loop moves through k: the stage's first byte
// and the panel's bytes from there, moved by one stage's step with additions only. records() clamps the bytes to
// [0, 2^31 - 1] exactly as Mem::resource does, from the 32-bit halves (the scalar unit has no signed 64-bit compare,
// and one on the vector unit costs an issue slot between MFMAs). walk(st) equals Loader::resource(st).
struct Walk {
  const char* at;
  std::int64_t left, step;
  CAIRN_HD unsigned records() const {
    const std::uint32_t hi = std::uint32_t(std::uint64_t(left) >> 32), lo = std::uint32_t(left);
    return std::int32_t(hi) < 0 ? 0u : (hi != 0u || lo > 0x7fffffffu ? 0x7fffffffu : lo);
  }
  CAIRN_HD void advance() {
    at += step;
    left -= step;
  }
};
template<class Sh, bool KMAJOR> CAIRN_HD Walk walk(const char* panel, std::int64_t bytes, std::int64_t ld, int st) {
  const std::int64_t step = KMAJOR ? std::int64_t(Sh::ROW) : std::int64_t(Sh::BK) * ld * Sh::ES;
  return Walk{panel + st * step, bytes - st * step, step};
}

// mnmajor_fragment(n0, s, h, l) - mnmajor_fragment(n0, 0, 0, l): the same for every lane and n0, because k-step s
// and half h move the k row by a multiple of the swizzle's period (4 rows of 16-bit elements, 8 of bytes). So a
// lane's transpose reads of one column block share one address register and differ by this immediate.
template<int ES, int R> constexpr int mnmajor_step(int s, int h) {
  return (ES == 2 ? 16 * s + 4 * h : 32 * s + 8 * h) * R * ES;
}

// The transpose reads as the hardware performs them, for the simulator: 16-lane groups, lane q of a group supplies
// 8 bytes; for 16-bit elements row r of the 4 x 16 block is lanes 4r .. 4r+3 (4 elements each) and lane q receives
// column q; for bytes row r of the 8 x 16 block is lanes 2r, 2r+1 (8 bytes each) and lane q receives column q.
CAIRN_HD void transpose_read(const std::uint8_t* lds, const int addr[64], int es, std::uint8_t out[64][8]) {
  for(int g = 0; g < 4; ++g)
    for(int q = 0; q < 16; ++q) {
      const int lane = 16 * g + q;
      if(es == 2) {
        for(int r = 0; r < 4; ++r) {
          const int src = 16 * g + 4 * r + (q >> 2);  // the lane holding row r, column q
          const std::uint8_t* at = lds + addr[src] + 2 * (q & 3);
          out[lane][2 * r] = at[0];
          out[lane][2 * r + 1] = at[1];
        }
      } else {
        for(int r = 0; r < 8; ++r) {
          const int src = 16 * g + 2 * r + (q >> 3);
          out[lane][r] = lds[addr[src] + (q & 7)];
        }
      }
    }
}

}  // namespace cairn::pipe
