// The index arithmetic of the pipelined gfx950 GEMM (gemm_pipe.hip), written once for the kernel and for the host
// simulator (tests/sim/tile_sim.cpp).
//
// A workgroup of eight waves computes a BM x BN tile. Operand tiles cross from global memory straight into LDS
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

template<int BM_, int BN_, int ES_, int STAGES_> struct Shape {
  static constexpr int BM = BM_, BN = BN_, ES = ES_, STAGES = STAGES_;
  static constexpr int ROW = 64;             // bytes of k per operand row per stage
  static constexpr int BK = ROW / ES;        // k elements per stage: 32 or 64
  static constexpr int CE = 16 / ES;         // k elements per 16-byte chunk of a K-major row
  static constexpr int THREADS = 512, GROUP = 256;
  static constexpr int WTM = BM / 2, WTN = BN / 4;  // a wave's outputs: group g holds rows g * BM/2 ..
  static constexpr int FM = WTM / 32, FN = WTN / 32;
  static constexpr int STEPS = 2;            // MFMA k-steps per stage
  static constexpr int A_BYTES = BM * ROW, B_BYTES = BN * ROW, STAGE = A_BYTES + B_BYTES;
  static constexpr int LOADS_A = BM * 4 / GROUP, LOADS_B = BN * 4 / GROUP;  // 16-byte loads per thread per stage
  static_assert(BM % 64 == 0 && BN % 128 == 0, "whole 32 x 32 blocks for every wave");
  static_assert(STAGES >= 3 && STAGES * STAGE <= 160 * 1024, "the ring fits the CU's LDS");
};

// The 16-byte LDS slot load u of thread t (0..255 within its loading group) writes: 16 q bytes into the operand's
// stage, q = (4 u + wave) * 64 + lane.
CAIRN_HD int slot(int t, int u) { return (u * 4 + (t >> 6)) * 64 + (t & 63); }

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
      const int q = slot(gt, u);
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
  // Stage `st` of k into LDS at `dst` (this operand's part of the ring buffer).
  CAIRN_HD void issue(Mem& mem, const char* panel, std::int64_t bytes, std::int64_t ld, int st, int k, char* dst, int w) {
    const std::int64_t step = KMAJOR ? std::int64_t(st) * Sh::ROW : std::int64_t(st) * Sh::BK * ld * Sh::ES;
    const auto r = mem.resource(panel + step, bytes - step);
    const int k0 = st * Sh::BK;
    const bool tail = k0 + Sh::BK > k;
#pragma unroll
    for(int u = 0; u < LOADS; ++u) {
      const int o = tail && k0 + kidx[u] >= k ? cairn::tile::OUTSIDE : offset[u];
      mem.load_lds(r, dst + (4 * u + w) * 1024, o);
    }
  }
};

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
