// The GEMM tile's data movement, written once for the gfx950 kernel and for the host tile simulator
// (tests/sim/tile_sim.cpp): which 16-byte chunks each thread fetches, how a chunk lands in LDS (K-major rows with an
// XOR swizzle), the register transposes that turn M- or N-contiguous operands K-major, which LDS chunk each lane
// reads for an MFMA operand, and which output element each accumulator register holds.
//
// The reference runs one fixed tiling, 64 x 64 outputs over k steps of 32 through two shared-memory stages
// (src/cairn/runtime/cairn_tensor.hpp:46-104). This tiling is the gfx950 one: up to 256 x 256 outputs per workgroup
// of four 64-wide waves, k steps of 128 bytes (64 bf16/f16 or 128 int8), operands always K-major in LDS, fed to
// v_mfma_f32_32x32x16_{bf16,f16} or v_mfma_i32_32x32x32_i8.
//
// Every function here is plain integer arithmetic on indices and 32-bit words, so the simulator runs the very code
// the kernel runs.
#pragma once
#include <cstddef>
#include <cstdint>
#include <type_traits>

#if defined(__HIPCC__)
#define CAIRN_HD __host__ __device__ inline __attribute__((always_inline))
#else
#define CAIRN_HD inline
#endif

namespace cairn::tile {

// 16 bytes: one chunk of a K-major LDS row, and one MFMA operand register quad.
typedef std::uint32_t u32x4 __attribute__((vector_size(16)));
typedef std::uint32_t u32x2 __attribute__((vector_size(8)));

// How operands cross from global memory into LDS: as stored, or (the 8-bit floats) widened to f16 in registers
// between their load and their LDS store, exactly (every value of either format is an f16 value), so that they meet
// the f16 matrix core, as the reference widens them for its f16 tensor cores (src/cairn/runtime/cairn_tensor.hpp:
// 123-135).
constexpr int WIDEN_NONE = 0, WIDEN_E4M3 = 1, WIDEN_E5M2 = 2;

// One tile configuration. ES is the operand's element size in LDS, in bytes (2: bf16/f16 and the widened 8-bit
// floats, 1: int8); GS its size in global memory (1 for the widened 8-bit floats, else ES). A k-step is 128 bytes of
// every operand row in LDS (8 chunks of 16 bytes); an MFMA consumes 32 bytes of k (2 chunks): 16 bf16 or 32 int8.
template<int BM_, int BN_, int ES_, int W_ = WIDEN_NONE> struct Shape {
  static constexpr int BM = BM_, BN = BN_, ES = ES_, W = W_;
  static constexpr int GS = W_ == WIDEN_NONE ? ES_ : 1;
  static_assert(W_ == WIDEN_NONE || ES_ == 2, "the 8-bit floats widen to f16");
  static constexpr int ROW = 128;              // bytes of one operand row per k-step, in LDS
  static constexpr int CHUNKS = ROW / 16;      // 8
  static constexpr int BK = ROW / ES;          // k elements per k-step: 64 or 128
  static constexpr int CE = 16 / ES;           // k elements per chunk: 8 or 16
  static constexpr int THREADS = 256;          // four waves of 64
  static constexpr int WAVES_M = 2, WAVES_N = 2;
  static constexpr int WTM = BM / WAVES_M, WTN = BN / WAVES_N;  // a wave's outputs
  static constexpr int FM = WTM / 32, FN = WTN / 32;            // its 32 x 32 MFMA blocks
  static constexpr int STEPS = CHUNKS / 2;                      // MFMA k-steps per k-step: 4
  static constexpr int A_BYTES = BM * ROW, B_BYTES = BN * ROW;  // one stage of each operand in LDS
  static constexpr int STAGE = A_BYTES + B_BYTES;
  // K-major fetch: every row's 8 chunks, spread over the threads.
  static constexpr int KA = BM * CHUNKS / THREADS, KB = BN * CHUNKS / THREADS;
  // MN-major fetch: blocks of KR k-rows x 8 m- or n-columns, one per thread while they last.
  static constexpr int KR = CE;                // k rows per block: a transposed chunk holds KR k values
  static_assert(BM % 128 == 0 && BN % 128 == 0, "each wave holds whole 32 x 32 blocks of a 2 x 2 wave grid");
  static_assert(KA >= 1 && KB >= 1, "every thread fetches at least one chunk of each K-major operand");
};

// The swizzle of a K-major LDS row: chunk c of row r lives at physical chunk c ^ swizzle(r). Eight consecutive rows
// read at one chunk (an MFMA operand fetch), and the eight rows of one transposed block written at one chunk, each
// spread over all eight chunk positions, so a group of eight lanes touches every bank once.
CAIRN_HD int swizzle(int row) { return (row ^ (row >> 3)) & 7; }
CAIRN_HD int lds_offset(int row, int chunk) { return row * 128 + 16 * (chunk ^ swizzle(row)); }

// K-major fetch slot u of thread t: row t/8 + 32u, chunk t%8. Eight consecutive threads read one row's 128
// contiguous bytes.
struct Slot {
  int row, chunk;
};
CAIRN_HD Slot kmajor_slot(int t, int u) {
  const int q = u * 256 + t;
  return Slot{q >> 3, q & 7};
}

// MN-major block of thread t for an operand of R rows (BM or BN): k rows kb*KR .. kb*KR+KR-1, columns nb*8 .. +7.
// Threads 0..31 of a wave read 32 consecutive 8-column pieces of one k row. Threads past R/... hold no block.
struct Block {
  int kb, nb;
  bool live;
};
template<int R> CAIRN_HD Block mnmajor_block(int t) {
  constexpr int across = R / 8;  // 8-column pieces in a k row
  return Block{t / across, t % across, t < 8 * across};
}

// The 8 x 8 transpose of 16-bit elements: in[r] holds row r's 8 elements (two to a word, the lower element in the
// low half); out[j] holds column j's 8 elements in the same packing.
CAIRN_HD void transpose_b16(const u32x4 in[8], u32x4 out[8]) {
#pragma unroll
  for(int j = 0; j < 8; ++j)
#pragma unroll
    for(int e = 0; e < 4; ++e) {
      const std::uint32_t x = in[2 * e][j >> 1], y = in[2 * e + 1][j >> 1];
      out[j][e] = (j & 1) ? ((x >> 16) | (y & 0xffff0000u)) : ((x & 0xffffu) | (y << 16));
    }
}

// The 16 x 8 transpose of bytes: in[r] holds row r's 8 bytes (byte c of the pair is column c); out[j] holds
// column j's 16 bytes, row r at byte r.
CAIRN_HD void transpose_b8(const u32x2 in[16], u32x4 out[8]) {
#pragma unroll
  for(int j = 0; j < 8; ++j)
#pragma unroll
    for(int e = 0; e < 4; ++e) {
      const int w = j >> 2, s = 8 * (j & 3);
      const std::uint32_t b0 = (in[4 * e][w] >> s) & 0xffu, b1 = (in[4 * e + 1][w] >> s) & 0xffu;
      const std::uint32_t b2 = (in[4 * e + 2][w] >> s) & 0xffu, b3 = (in[4 * e + 3][w] >> s) & 0xffu;
      out[j][e] = b0 | (b1 << 8) | (b2 << 16) | (b3 << 24);
    }
}

// Eight 8-bit floats (byte e of the pair is element e) as eight f16 patterns (two to a word, the lower element in
// the low half), exactly. E5M2 is the top byte of the f16 of the same value. E4M3 goes through the hardware's packed
// conversion at scale 1 on the device (an f16 holds every E4M3 value, subnormals included) and through the same
// rebias in integer steps on the host (the simulator), its NaN to f16's quiet NaN.
CAIRN_HD std::uint16_t e4m3_as_f16(std::uint32_t x) {
  const std::uint32_t sign = (x & 0x80u) << 8, e = (x >> 3) & 15u, f = x & 7u;
  if(e == 15u && f == 7u) return std::uint16_t(sign | 0x7e00u);
  if(e == 0u) {
    if(f == 0u) return std::uint16_t(sign);
    const unsigned lead = f >= 4u ? 2u : (f >= 2u ? 1u : 0u);  // f * 2^-9 = 1.xx * 2^(lead - 9)
    return std::uint16_t(sign | ((lead + 6u) << 10) | ((f - (1u << lead)) << (10u - lead)));
  }
  return std::uint16_t(sign | ((e + 8u) << 10) | (f << 7));
}
template<int W> CAIRN_HD u32x4 widened(u32x2 raw) {
  u32x4 out;
#pragma unroll
  for(int h = 0; h < 2; ++h) {
    const std::uint32_t x = raw[h];
    if constexpr(W == WIDEN_E5M2) {
      out[2 * h] = ((x & 0xffu) << 8) | ((x & 0xff00u) << 16);
      out[2 * h + 1] = ((x >> 8) & 0xff00u) | (x & 0xff000000u);
    } else {
#if defined(__HIP_DEVICE_COMPILE__)
      out[2 * h] = __builtin_bit_cast(std::uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(x, 1.0f, false));
      out[2 * h + 1] = __builtin_bit_cast(std::uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(x, 1.0f, true));
#else
      out[2 * h] = std::uint32_t(e4m3_as_f16(x & 0xffu)) | (std::uint32_t(e4m3_as_f16((x >> 8) & 0xffu)) << 16);
      out[2 * h + 1] = std::uint32_t(e4m3_as_f16((x >> 16) & 0xffu)) | (std::uint32_t(e4m3_as_f16(x >> 24)) << 16);
#endif
    }
  }
  return out;
}

// The LDS chunk lane l reads for MFMA k-step s of the 32-row block starting at `row0`: row row0 + l%32, chunk
// 2s + l/32. Lanes 0..31 hold the first 32 bytes of k, lanes 32..63 the next; both operands use the same split, so
// each product pairs one k with itself whatever order the matrix core adds them in.
CAIRN_HD int fragment_offset(int row0, int s, int lane) { return lds_offset(row0 + (lane & 31), 2 * s + (lane >> 5)); }

// The accumulator of one 32 x 32 block, with the B fragment as the MFMA's first operand and the A fragment as its
// second: register r of lane l is output (m, n) = (l%32, 8*(r/4) + 4*(l/32) + r%4). Registers 4q..4q+3 are four
// consecutive columns of one row, so each lane stores 16 (f32) or 8 (bf16) contiguous bytes.
CAIRN_HD int acc_m(int lane) { return lane & 31; }
CAIRN_HD int acc_n(int lane, int q) { return 8 * q + 4 * (lane >> 5); }

// The output tile workgroup b computes. The dispatcher hands workgroups to the 8 XCDs round-robin (b on XCD b % 8)
// and each XCD has its own L2, so ids are first remapped to give each XCD a contiguous run; ids then walk `group`
// tile rows at a time, column by column, so the tiles an XCD holds at once share their a and b panels. A bijection
// of [0, tiles_m * tiles_n) onto the tiles.
// xcd_order: workgroup b of `count` to its id (a bijection of [0, count)); tile_at: an id to its tile.
CAIRN_HD int xcd_order(int b, int count) { return count % 8 == 0 ? (b % 8) * (count / 8) + b / 8 : b; }
CAIRN_HD void tile_at(int id, int tiles_m, int tiles_n, int group, int& tm, int& tn) {
  const int per = group * tiles_n;
  const int first = (id / per) * group;
  const int rows = tiles_m - first < group ? tiles_m - first : group;
  const int local = id - (id / per) * per;
  tm = first + local % rows;
  tn = local / rows;
}
CAIRN_HD void tile_of(int b, int tiles_m, int tiles_n, int group, int& tm, int& tn) {
  tile_at(xcd_order(b, tiles_m * tiles_n), tiles_m, tiles_n, group, tm, tn);
}

// The split last round. Where the tiles are not a whole number of rounds of the machine, each XCD's block of ids
// (xcd_order: `block` ids an XCD, `xcds` blocks) keeps its first `first` ids, whole rounds of its CUs, for the
// whole-tile pass, and shares its remaining `tiles` ids along k among `units` workgroups that run on the same XCD,
// so that the panels its tiles share stay in its L2: those tiles' stages, `stages` a tile, laid end to end, unit v
// of the XCD taking the `quota` stages from v quota on. A unit's run stays within two tiles (quota <= stages), so it
// writes at most two partial tiles. A fixup pass then adds each tile's partials in the order of their units (their
// k order, so the bits do not depend on timing) and applies the epilogue.
//
// Workgroup b of the whole-tile pass (xcds * first of them) runs id whole_id(b); workgroup u of the split pass
// (xcds * units) is unit u / xcds of XCD u % xcds (the dispatcher hands workgroup u to XCD u % 8), and its partial
// tiles go to slots 2 u and 2 u + 1.
struct Split {
  int first = 0;   // ids of an XCD's block that the whole-tile pass runs
  int tiles = 0;   // ids of an XCD's block shared along k (0: no split)
  int stages = 0;  // k stages a tile
  int quota = 0;   // stages a unit
  int units = 0;   // units an XCD
  int xcds = 1;    // XCD blocks
  int block = 0;   // ids an XCD's block
};
CAIRN_HD int whole_id(const Split& s, int b) { return (b % s.xcds) * s.block + b / s.xcds; }
// The id of split tile t of XCD x.
CAIRN_HD int split_id(const Split& s, int x, int t) { return x * s.block + s.first + t; }
// Segment j (0 or 1) of unit v of an XCD: its tile (0 .. tiles - 1 of the XCD's) and its stages [s0, s1) within
// that tile; false where the unit has no such segment.
CAIRN_HD bool split_segment(const Split& s, int v, int j, int& tile, int& s0, int& s1) {
  const long long total = (long long)s.tiles * s.stages;
  long long g0 = (long long)v * s.quota;
  const long long g1 = g0 + s.quota < total ? g0 + s.quota : total;
  if(g0 >= g1) return false;
  if(j == 1) {
    const long long next = (g0 / s.stages + 1) * s.stages;  // the start of the next tile
    if(next >= g1) return false;
    g0 = next;
  }
  tile = int(g0 / s.stages);
  const long long end = (long long)(tile + 1) * s.stages < g1 ? (long long)(tile + 1) * s.stages : g1;
  s0 = int(g0 - (long long)tile * s.stages);
  s1 = int(end - (long long)tile * s.stages);
  return true;
}
// The units of an XCD whose runs meet its tile t (first .. last, in k order), and the slot unit v of XCD x wrote its
// part of tile t to.
CAIRN_HD void split_units_of(const Split& s, int t, int& first, int& last) {
  first = int((long long)t * s.stages / s.quota);
  last = int(((long long)(t + 1) * s.stages - 1) / s.quota);
}
CAIRN_HD int split_slot(const Split& s, int x, int t, int v) {
  return 2 * (v * s.xcds + x) + ((long long)v * s.quota < (long long)t * s.stages ? 1 : 0);
}

constexpr int OUTSIDE = 0x7fffffff;  // a byte offset past every resource: the load reads zero

// The first byte of an operand panel and the bytes from there to the end of the stored matrix. The panel holds the
// operand's rows first .. first + R - 1 (K-major: stored rows; MN-major: stored columns), at k = 0.
struct Panel {
  std::int64_t start, bytes;
};
CAIRN_HD Panel panel(bool kmajor, int first, int total, int k, std::int64_t ld, int es) {
  if(kmajor) return Panel{std::int64_t(first) * ld * es, (std::int64_t(total - 1) * ld + k) * es - std::int64_t(first) * ld * es};
  return Panel{std::int64_t(first) * es, (std::int64_t(k - 1) * ld + total) * es - std::int64_t(first) * es};
}

// One operand's share of one k-step: fetched into registers through Mem (buffer loads on the device, checked reads
// in the simulator), then written into a stage of LDS. R rows of the operand start at `first` of `total`.
// Mem::Rsrc Mem::resource(const char* base, int64 bytes); Mem::load16(Rsrc, int) -> u32x4; Mem::load8 -> u32x2.
template<class Sh, int R, bool KMAJOR, class Mem> struct Operand;

// K-contiguous rows: slot u of thread t is row kmajor_slot(t,u).row, chunk .chunk; 16-byte loads (8-byte ones of
// the 8-bit floats that widen to a 16-byte chunk).
template<class Sh, int R, class Mem> struct Operand<Sh, R, true, Mem> {
  static constexpr int SLOTS = R * Sh::CHUNKS / Sh::THREADS;
  using Raw = typename std::conditional<Sh::GS == Sh::ES, u32x4, u32x2>::type;
  Raw v[SLOTS];
  int offset[SLOTS];  // from the panel's start, or OUTSIDE for rows past `total`
  CAIRN_HD void setup(int t, int first, int total, std::int64_t ld) {
#pragma unroll
    for(int u = 0; u < SLOTS; ++u) {
      const Slot s = kmajor_slot(t, u);
      offset[u] = first + s.row < total ? int(s.row * ld * Sh::GS) + Sh::CE * Sh::GS * s.chunk : OUTSIDE;
    }
  }
  // k-step kt: the panel advanced by kt * BK elements; chunks at or past k read nothing.
  CAIRN_HD void fetch(Mem& mem, const char* base, const Panel& p, std::int64_t, int kt, int k, int t) {
    const std::int64_t step = std::int64_t(kt) * Sh::BK * Sh::GS;
    const auto r = mem.resource(base + p.start + step, p.bytes - step);
    const int k0 = kt * Sh::BK;
    const bool tail = k0 + Sh::BK > k;
#pragma unroll
    for(int u = 0; u < SLOTS; ++u) {
      int o = offset[u];
      if(tail && k0 + kmajor_slot(t, u).chunk * Sh::CE >= k) o = OUTSIDE;
      if constexpr(Sh::GS == Sh::ES) v[u] = mem.load16(r, o);
      else v[u] = mem.load8(r, o);
    }
  }
  template<class Lds> CAIRN_HD void store(Lds& lds, int stage, int t) const {
#pragma unroll
    for(int u = 0; u < SLOTS; ++u) {
      const Slot s = kmajor_slot(t, u);
      if constexpr(Sh::GS == Sh::ES) lds.write16(stage + lds_offset(s.row, s.chunk), v[u]);
      else lds.write16(stage + lds_offset(s.row, s.chunk), widened<Sh::W>(v[u]));
    }
  }
};

// M- or N-contiguous rows: this thread's block of KR k rows x 8 columns, transposed into 8 K-major chunks (the 8-bit
// floats that widen: each k row's 8 bytes widened to 8 f16, then transposed as 16-bit elements).
template<class Sh, int R, class Mem> struct Operand<Sh, R, false, Mem> {
  static constexpr int KR = Sh::KR;
  using Piece = typename std::conditional<Sh::GS == 2, u32x4, u32x2>::type;
  Piece v[KR];
  int col;    // byte offset of this thread's 8 columns in a stored row, or OUTSIDE
  bool live;  // holds a block
  CAIRN_HD void setup(int t, int first, int total, std::int64_t) {
    const Block b = mnmajor_block<R>(t);
    live = b.live;
    col = b.live && first + 8 * b.nb < total ? 8 * b.nb * Sh::GS : OUTSIDE;
  }
  // k-step kt: the panel advanced by kt * BK stored rows; rows at or past k read nothing.
  CAIRN_HD void fetch(Mem& mem, const char* base, const Panel& p, std::int64_t ld, int kt, int k, int t) {
    if(!live) return;
    const int k0 = kt * Sh::BK;
    const std::int64_t step = std::int64_t(k0) * ld * Sh::GS;
    const auto r = mem.resource(base + p.start + step, p.bytes - step);
    const int kb = mnmajor_block<R>(t).kb;
#pragma unroll
    for(int q = 0; q < KR; ++q) {
      const int row = kb * KR + q;
      const int o = col == OUTSIDE || k0 + row >= k ? OUTSIDE : int(row * ld * Sh::GS) + col;
      if constexpr(Sh::GS == 2) v[q] = mem.load16(r, o);
      else v[q] = mem.load8(r, o);
    }
  }
  template<class Lds> CAIRN_HD void store(Lds& lds, int stage, int t) const {
    if(!live) return;
    const Block b = mnmajor_block<R>(t);
    u32x4 out[8];
    if constexpr(Sh::GS == 2) {
      transpose_b16(v, out);
    } else if constexpr(Sh::ES == 2) {
      u32x4 wide[8];
#pragma unroll
      for(int q = 0; q < 8; ++q) wide[q] = widened<Sh::W>(v[q]);
      transpose_b16(wide, out);
    } else {
      transpose_b8(v, out);
    }
#pragma unroll
    for(int j = 0; j < 8; ++j) lds.write16(stage + lds_offset(8 * b.nb + j, b.kb), out[j]);
  }
};

}  // namespace cairn::tile
