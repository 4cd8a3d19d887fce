// The gfx950 MFMA tile run on the host: every thread's fetches, transposes and LDS writes through the very code the
// kernel runs (cairn_amd/csrc/tile.hpp), every lane's fragment reads, a model of the matrix core, and the epilogue's
// output mapping. It holds the kernel's index arithmetic to four rules, for every layout, tile shape and operand size,
// on shapes with tails in every direction and padded leading dimensions:
//
//   1. every global load the kernel makes either lies wholly inside its matrix's allocation or is one the hardware
//      turns into zeros (an offset past the buffer resource), and no load straddles the resource's end;
//   2. every 16-byte chunk of an LDS stage is written exactly once per k-step, inside the stage;
//   3. every output element is written exactly once, and none outside the matrix;
//   4. the outputs equal the exact product (values chosen so every sum is exact), old values added.
//
// The widened 8-bit float shapes load 8 bytes of an operand where the others load 16 and widen them to f16 between
// the load and the LDS store (the host side of tile.hpp's widened), so rules 1-4 hold their loads and tails too.
//
// The matrix-core model: lane l supplies row l%32 of its operand and 16 bytes of k (chunk 2s + l/32); the output of
// register r of lane l is row 8(r/4) + 4(l/32) + r%4 of the first operand, column l%32 of the second. The GPU tests
// check the model against the hardware; this program checks everything around it. Mirrors, in spirit, the
// reference's host run of its device tile (tests/runtime/tensor_runtime.cpp).
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>
#include <utility>
#include "pipe.hpp"
#include "tile.hpp"

using namespace cairn::tile;

namespace {

int failures = 0;
#define FAIL(...)                 \
  do {                            \
    std::printf(__VA_ARGS__);     \
    std::printf("\n");            \
    ++failures;                   \
    return;                       \
  } while(0)

std::uint64_t mix(std::uint64_t x) {
  x ^= x >> 31;
  x *= 0x7fb5d329728ea185ULL;
  x ^= x >> 27;
  x *= 0x94d049bb133111ebULL;
  x ^= x >> 29;
  return x;
}

// Checked memory: a load must lie inside the resource or be wholly past it; a load inside the resource must lie
// inside the allocation the matrix came from.
struct HostMem {
  const char* lo;
  const char* hi;
  bool bad = false;
  struct Rsrc {
    const char* base;
    std::int64_t bytes;
  };
  Rsrc resource(const char* base, std::int64_t bytes) {
    return Rsrc{base, bytes < 0 ? 0 : (bytes > 0x7fffffffLL ? 0x7fffffffLL : bytes)};
  }
  Rsrc resource(const cairn::pipe::Walk& w) { return Rsrc{w.at, std::int64_t(w.records())}; }
  template<int N> void read(Rsrc r, int off, std::uint32_t* out) {
    std::memset(out, 0, N);
    if(off < 0) bad = true;
    if(off >= r.bytes) return;  // the hardware's zeros
    if(std::int64_t(off) + N > r.bytes) bad = true;  // straddles the resource's end
    const char* at = r.base + off;
    if(at < lo || at + N > hi) {
      bad = true;
      return;
    }
    std::memcpy(out, at, N);
  }
  u32x4 load16(Rsrc r, int off) {
    std::uint32_t w[4];
    read<16>(r, off, w);
    return u32x4{w[0], w[1], w[2], w[3]};
  }
  u32x2 load8(Rsrc r, int off) {
    std::uint32_t w[2];
    read<8>(r, off, w);
    return u32x2{w[0], w[1]};
  }
};

struct HostLds {
  std::vector<std::uint8_t> bytes;
  std::vector<int> writes;  // per 16-byte chunk
  bool bad = false;
  explicit HostLds(int size) : bytes(size), writes(size / 16) {}
  void write16(int off, u32x4 v) {
    if(off < 0 || off % 16 || off + 16 > int(bytes.size())) {
      bad = true;
      return;
    }
    std::memcpy(&bytes[off], &v, 16);
    ++writes[off / 16];
  }
};

// Operand values: bf16 (a multiple of 1/16 in [-1.875, 1.875]) or int8 in [-127, 127]; the element is written into
// the stored matrix at `at`.
template<int ES> double value_of(const std::vector<std::uint8_t>& m, std::int64_t at) {
  if constexpr(ES == 2) {
    std::uint16_t b;
    std::memcpy(&b, &m[at * 2], 2);
    const std::uint32_t u = std::uint32_t(b) << 16;
    float f;
    std::memcpy(&f, &u, 4);
    return f;
  } else {
    return double(std::int8_t(m[at]));
  }
}
template<int ES> void put(std::vector<std::uint8_t>& m, std::int64_t at, std::uint64_t h) {
  if constexpr(ES == 2) {
    const float f = float(std::int64_t(h % 61) - 30) / 16.0f;  // exact in bf16
    std::uint32_t u;
    std::memcpy(&u, &f, 4);
    const std::uint16_t b = std::uint16_t(u >> 16);
    std::memcpy(&m[at * 2], &b, 2);
  } else {
    m[at] = std::uint8_t(std::int8_t(std::int64_t(h % 255) - 127));
  }
}
// A chunk's elements as values.
template<int ES> void decode(const std::uint8_t* chunk, double* out) {
  for(int e = 0; e < 16 / ES; ++e) {
    if constexpr(ES == 2) {
      std::uint16_t b;
      std::memcpy(&b, chunk + 2 * e, 2);
      const std::uint32_t u = std::uint32_t(b) << 16;
      float f;
      std::memcpy(&f, &u, 4);
      out[e] = f;
    } else {
      out[e] = double(std::int8_t(chunk[e]));
    }
  }
}

// The 8-bit floats' values, from their fields (E4M3: bias 7, no infinities, S.1111.111 NaN; E5M2: bias 15, IEEE
// specials), and f16's, for the widened shapes' LDS chunks.
double f8_value(std::uint8_t x, int w) {
  const int sign = x & 0x80 ? -1 : 1;
  const int mbits = w == WIDEN_E4M3 ? 3 : 2, bias = w == WIDEN_E4M3 ? 7 : 15;
  const int e = (x & 0x7f) >> mbits, f = x & ((1 << mbits) - 1);
  if(w == WIDEN_E4M3 && e == 15 && f == 7) return std::nan("");
  if(w == WIDEN_E5M2 && e == 31) return f ? std::nan("") : sign * INFINITY;
  const double mant = e ? 1.0 + std::ldexp(double(f), -mbits) : std::ldexp(double(f), -mbits);
  return sign * std::ldexp(mant, (e ? e : 1) - bias);
}
double f16_value(std::uint16_t h) {
  const int sign = h & 0x8000 ? -1 : 1, e = (h >> 10) & 31, f = h & 1023;
  if(e == 31) return f ? std::nan("") : sign * INFINITY;
  return sign * std::ldexp(e ? 1.0 + std::ldexp(double(f), -10) : std::ldexp(double(f), -10), (e ? e : 1) - 15);
}
// An operand's element: its size in memory (GS) and in LDS (ES), its value in memory and in an LDS chunk. The widened
// 8-bit floats draw from every finite E4M3 pattern and from E5M2's with exponents 6 .. 25 (2^-9 .. 1.75 2^10), ranges
// whose products' sums over k of a few thousand are exact in a double.
template<int ES, int W> struct Codec {
  static constexpr int GS = W == WIDEN_NONE ? ES : 1;
  static double value(const std::vector<std::uint8_t>& m, std::int64_t at) {
    if constexpr(W == WIDEN_NONE) return value_of<ES>(m, at);
    else return f8_value(m[at], W);
  }
  static void put(std::vector<std::uint8_t>& m, std::int64_t at, std::uint64_t h) {
    if constexpr(W == WIDEN_NONE) {
      ::put<ES>(m, at, h);
    } else if constexpr(W == WIDEN_E4M3) {
      std::uint8_t x = std::uint8_t(h % 254);
      m[at] = x >= 0x7f ? std::uint8_t(x + 1) : x;  // 0x7f (NaN) skipped; 0xff never drawn
    } else {
      const std::uint8_t e = std::uint8_t(6 + (h >> 8) % 20), f = std::uint8_t(h & 3), sign = std::uint8_t(h & 4 ? 0x80 : 0);
      m[at] = std::uint8_t(sign | (e << 2) | f);
    }
  }
  static void chunk(const std::uint8_t* c, double* out) {
    if constexpr(W == WIDEN_NONE) {
      decode<ES>(c, out);
    } else {
      for(int e = 0; e < 8; ++e) {
        std::uint16_t h;
        std::memcpy(&h, c + 2 * e, 2);
        out[e] = f16_value(h);
      }
    }
  }
};

// The host widening (the simulator's stand-in for the hardware conversion) gives every pattern's own value: E4M3 and
// E5M2 are f16 values, so the widened f16 must decode to the same number (NaN to a NaN).
void widening_is_exact() {
  for(int w : {WIDEN_E4M3, WIDEN_E5M2}) {
    for(int x = 0; x < 256; ++x) {
      const u32x2 raw{std::uint32_t(x) * 0x01010101u, std::uint32_t(x) * 0x01010101u};
      const u32x4 out = w == WIDEN_E4M3 ? widened<WIDEN_E4M3>(raw) : widened<WIDEN_E5M2>(raw);
      for(int e = 0; e < 8; ++e) {
        const std::uint16_t h = std::uint16_t(out[e / 2] >> (16 * (e % 2)));
        const double want = f8_value(std::uint8_t(x), w), got = f16_value(h);
        if(std::isnan(want) ? !std::isnan(got) : (got != want || std::signbit(got) != std::signbit(want))) {
          std::printf("widen %s 0x%02x: element %d is f16 0x%04x = %.9g, want %.9g\n", w == WIDEN_E4M3 ? "e4m3" : "e5m2",
                      x, e, h, got, want);
          ++failures;
          return;
        }
      }
    }
    // Distinct bytes land in their own elements, in order.
    const u32x2 ramp{0x43424140u, 0x47464544u};
    const u32x4 r = w == WIDEN_E4M3 ? widened<WIDEN_E4M3>(ramp) : widened<WIDEN_E5M2>(ramp);
    for(int e = 0; e < 8; ++e) {
      const std::uint16_t h = std::uint16_t(r[e / 2] >> (16 * (e % 2)));
      if(f16_value(h) != f8_value(std::uint8_t(0x40 + e), w)) {
        std::printf("widen: element %d out of place\n", e);
        ++failures;
        return;
      }
    }
  }
}

template<int BM, int BN, int ES, bool TA, bool TB, int W = WIDEN_NONE> void run(int m, int n, int k, int pad, int group) {
  using Sh = Shape<BM, BN, ES, W>;
  using V = Codec<ES, W>;
  constexpr int GS = V::GS;
  constexpr bool AK = !TA, BK_ = TB;
  const char* lay = TA ? (TB ? "TT" : "TN") : (TB ? "NT" : "NN");
  // Stored matrices, padded: a is m x k (TA: k x m), b is k x n (TB: n x k).
  const std::int64_t lda = (TA ? m : k) + pad, ldb = (TB ? k : n) + pad, ldc = n + pad;
  const std::int64_t arows = TA ? k : m, brows = TB ? n : k;
  const std::int64_t abytes = std::max<std::int64_t>(1, ((arows ? arows - 1 : 0) * lda + (TA ? m : k)) * GS);
  const std::int64_t bbytes = std::max<std::int64_t>(1, ((brows ? brows - 1 : 0) * ldb + (TB ? k : n)) * GS);
  std::vector<std::uint8_t> A(abytes, 0x7f), B(bbytes, 0x7f);  // padding: 0x7f7f is a huge bf16, 127 an int8
  for(std::int64_t r = 0; r < arows; ++r)
    for(int q = 0; q < (TA ? m : k); ++q) V::put(A, r * lda + q, mix(11 + r * 7919 + q));
  for(std::int64_t r = 0; r < brows; ++r)
    for(int q = 0; q < (TB ? k : n); ++q) V::put(B, r * ldb + q, mix(23 + r * 104729 + q));
  auto a_at = [&](int i, int p) { return TA ? std::int64_t(p) * lda + i : std::int64_t(i) * lda + p; };
  auto b_at = [&](int p, int j) { return TB ? std::int64_t(j) * ldb + p : std::int64_t(p) * ldb + j; };

  std::vector<double> C(std::size_t(m) * ldc), old(std::size_t(m) * ldc);
  std::vector<int> written(std::size_t(m) * ldc);
  for(std::size_t e = 0; e < C.size(); ++e) C[e] = old[e] = double(std::int64_t(mix(99 + e) % 9) - 4) / 4.0;

  const int tiles_m = (m + BM - 1) / BM, tiles_n = (n + BN - 1) / BN, total = tiles_m * tiles_n;
  std::vector<int> seen(total);
  HostMem mem_a{reinterpret_cast<const char*>(A.data()), reinterpret_cast<const char*>(A.data()) + A.size()};
  HostMem mem_b{reinterpret_cast<const char*>(B.data()), reinterpret_cast<const char*>(B.data()) + B.size()};
  for(int wg = 0; wg < total; ++wg) {
    int tm, tn;
    tile_of(wg, tiles_m, tiles_n, group, tm, tn);
    if(tm < 0 || tm >= tiles_m || tn < 0 || tn >= tiles_n) FAIL("%s tile_of(%d) = (%d, %d) off the grid", lay, wg, tm, tn);
    ++seen[tm * tiles_n + tn];
    const int row0 = tm * BM, col0 = tn * BN;
    const Panel pa = panel(AK, row0, m, k, lda, GS), pb = panel(BK_, col0, n, k, ldb, GS);
    std::vector<Operand<Sh, BM, AK, HostMem>> fa(Sh::THREADS);
    std::vector<Operand<Sh, BN, BK_, HostMem>> fb(Sh::THREADS);
    for(int t = 0; t < Sh::THREADS; ++t) {
      fa[t].setup(t, row0, m, lda);
      fb[t].setup(t, col0, n, ldb);
    }
    std::vector<double> acc(static_cast<std::size_t>(BM * BN), 0.0);  // by output (row, column) of the tile
    const int steps = (k + Sh::BK - 1) / Sh::BK;
    for(int kt = 0; kt < steps; ++kt) {
      HostLds lds(Sh::STAGE);
      for(int t = 0; t < Sh::THREADS; ++t) {
        fa[t].fetch(mem_a, reinterpret_cast<const char*>(A.data()), pa, lda, kt, k, t);
        fb[t].fetch(mem_b, reinterpret_cast<const char*>(B.data()), pb, ldb, kt, k, t);
        fa[t].store(lds, 0, t);
        fb[t].store(lds, Sh::A_BYTES, t);
      }
      if(mem_a.bad || mem_b.bad) FAIL("%s %dx%d es=%d %dx%dx%d: a global load outside its matrix", lay, BM, BN, ES, m, n, k);
      if(lds.bad) FAIL("%s %dx%d: an LDS write off the stage", lay, BM, BN);
      for(int c = 0; c < Sh::STAGE / 16; ++c)
        if(lds.writes[c] != 1) FAIL("%s %dx%d es=%d: LDS chunk %d written %d times", lay, BM, BN, ES, c, lds.writes[c]);
      // The matrix core, wave by wave: first operand the B block (rows = n), second the A block (columns = m).
      for(int w = 0; w < 4; ++w) {
        const int wm = w / Sh::WAVES_N, wn = w % Sh::WAVES_N;
        for(int s = 0; s < Sh::STEPS; ++s)
          for(int i = 0; i < Sh::FM; ++i)
            for(int j = 0; j < Sh::FN; ++j) {
              double P[32][32], Q[32][32];  // P[row][kk], Q[kk][col], kk over this step's 32 bytes of k
              constexpr int CE = 16 / ES;
              for(int l = 0; l < 64; ++l) {
                double pb_[16], qa_[16];
                V::chunk(&lds.bytes[Sh::A_BYTES + fragment_offset(wn * Sh::WTN + 32 * j, s, l)], pb_);
                V::chunk(&lds.bytes[fragment_offset(wm * Sh::WTM + 32 * i, s, l)], qa_);
                for(int e = 0; e < CE; ++e) {
                  P[l & 31][(l >> 5) * CE + e] = pb_[e];
                  Q[(l >> 5) * CE + e][l & 31] = qa_[e];
                }
              }
              for(int l = 0; l < 64; ++l)
                for(int r = 0; r < 16; ++r) {
                  const int prow = 8 * (r / 4) + 4 * (l / 32) + r % 4, qcol = l % 32;
                  double sum = 0;
                  for(int kk = 0; kk < 2 * CE; ++kk) sum += P[prow][kk] * Q[kk][qcol];
                  // Output mapping of tile.hpp: lane l, quad q = r/4, element e = r%4.
                  const int mm = wm * Sh::WTM + 32 * i + acc_m(l);
                  const int nn = wn * Sh::WTN + 32 * j + acc_n(l, r / 4) + r % 4;
                  if(mm != wm * Sh::WTM + 32 * i + qcol || nn != wn * Sh::WTN + 32 * j + prow)
                    FAIL("%s: accumulator mapping disagrees with the matrix-core model", lay);
                  acc[std::size_t(mm) * BN + nn] += sum;
                }
            }
      }
    }
    // Epilogue: every output of the tile inside the matrix, once.
    for(int w = 0; w < 4; ++w) {
      const int wm = w / Sh::WAVES_N, wn = w % Sh::WAVES_N;
      for(int i = 0; i < Sh::FM; ++i)
        for(int j = 0; j < Sh::FN; ++j)
          for(int l = 0; l < 64; ++l)
            for(int q = 0; q < 4; ++q) {
              const int mm = wm * Sh::WTM + 32 * i + acc_m(l), nn0 = wn * Sh::WTN + 32 * j + acc_n(l, q);
              const int gm = row0 + mm, gn = col0 + nn0;
              if(gm >= m || gn >= n) continue;
              if(gn + 3 >= n + 3 && n % 4) FAIL("%s: a quad straddles n", lay);
              for(int e = 0; e < 4; ++e) {
                const std::size_t at = std::size_t(gm) * ldc + gn + e;
                C[at] = old[at] + acc[std::size_t(mm) * BN + nn0 + e];
                ++written[at];
              }
            }
    }
  }
  for(int id = 0; id < total; ++id)
    if(seen[id] != 1) FAIL("%s: tile %d computed %d times", lay, id, seen[id]);
  for(int i = 0; i < m; ++i)
    for(int j = 0; j < n; ++j) {
      double want = old[std::size_t(i) * ldc + j];
      double exact = 0;
      for(int p = 0; p < k; ++p) exact += V::value(A, a_at(i, p)) * V::value(B, b_at(p, j));
      want += exact;
      const std::size_t at = std::size_t(i) * ldc + j;
      if(written[at] != 1) FAIL("%s %dx%d es=%d %dx%dx%d: output (%d,%d) written %d times", lay, BM, BN, ES, m, n, k, i, j, written[at]);
      if(C[at] != want)
        FAIL("%s %dx%d es=%d %dx%dx%d pad %d: output (%d,%d) is %.9g, exact %.9g", lay, BM, BN, ES, m, n, k, pad, i, j,
             C[at], want);
    }
}

// ---------------------------------------------------------------- the LDS-ring kernels' index math (pipe.hpp; wave.hpp, and eight waves a workgroup)

bool bad_read = false;
bool conflict = false;
bool stepped_off = false;
// gfx950 LDS: 64 banks of 4 bytes. A ds_read_b128 is served 16 lanes a clock, a 64-bit read 32 lanes a clock; a
// phase without conflicts touches each bank once.
void check_banks(const int addr[64], int bytes) {
  const int lanes = 256 / bytes;
  for(int p0 = 0; p0 < 64; p0 += lanes) {
    int seen[64] = {};
    for(int l = p0; l < p0 + lanes; ++l)
      for(int w = 0; w < bytes / 4; ++w) ++seen[(addr[l] / 4 + w) % 64];
    for(int b = 0; b < 64; ++b)
      if(seen[b] != 1) conflict = true;
  }
}
template<int ES, int R> int frag_mn(int n0, int s, int h, int l) { return cairn::pipe::mnmajor_fragment<ES, R>(n0, s, h, l); }

// The direct loads: lane `lane` of the issuing wave writes 16 bytes at the wave's LDS base + 16 lane.
struct HostDma {
  HostMem* mem;
  HostLds* lds;
  const std::uint8_t* ring;  // lds->bytes.data()
  int lane = 0;
  using Rsrc = HostMem::Rsrc;
  Rsrc resource(const char* base, std::int64_t bytes) { return mem->resource(base, bytes); }
  Rsrc resource(const cairn::pipe::Walk& w) { return mem->resource(w); }
  void load_lds(Rsrc r, char* wave_base, int offset) {
    const u32x4 v = mem->load16(r, offset);
    lds->write16(int(reinterpret_cast<std::uint8_t*>(wave_base) - ring) + 16 * lane, v);
  }
  // M0 and the immediate offset: the lane's offset register holds offset - 1024 U, which must not go below zero.
  char* m0 = nullptr;
  bool negative = false;
  void set_base(char* base) { m0 = base; }
  template<int U> void load_lds_imm(Rsrc r, int offset) {
    if(offset != OUTSIDE && offset - 1024 * U < 0) negative = true;
    load_lds(r, m0 + 1024 * U, offset);
  }
};

template<class L, class D, class R, std::size_t... U>
void imm_loads(const L& l, D& d, const R& r, int st, int k, std::index_sequence<U...>) {
  (l.template load_imm<int(U)>(d, r, st, k), ...);
}
// The main loop's loads of a stage that ends at or before k (or lies past the last): no per-chunk k check.
template<class L, class D, class R, std::size_t... U>
void steady_loads(const L& l, D& d, const R& r, std::index_sequence<U...>) {
  (l.template load_steady<int(U)>(d, r), ...);
}
// The walked resource of stage st (the main loop's) must be the one Loader::resource computes.
template<class Sh, bool KMAJOR>
HostMem::Rsrc walked(HostMem& mem, const char* panel, std::int64_t bytes, std::int64_t ld, int st) {
  cairn::pipe::Walk w = cairn::pipe::walk<Sh, KMAJOR>(panel, bytes, ld, st > 2 ? st - 2 : 0);
  for(int i = st > 2 ? st - 2 : 0; i < st; ++i) w.advance();
  const HostMem::Rsrc got = mem.resource(w), want = mem.resource(panel + (KMAJOR ? std::int64_t(st) * Sh::ROW : std::int64_t(st) * Sh::BK * ld * Sh::ES),
                                                                 bytes - (KMAJOR ? std::int64_t(st) * Sh::ROW : std::int64_t(st) * Sh::BK * ld * Sh::ES));
  if(got.base != want.base || got.bytes != want.bytes) {
    std::printf("walk: stage %d resource differs from Loader::resource\n", st);
    ++failures;
  }
  return got;
}

template<class Sh, bool TA, bool TB> void run_pipe(int m, int n, int k, int pad, int group) {
  constexpr int BM = Sh::BM, BN = Sh::BN, ES = Sh::ES;
  constexpr bool AK = !TA, BKM = TB;
  const char* lay = TA ? (TB ? "TT" : "TN") : (TB ? "NT" : "NN");
  const std::int64_t lda = (TA ? m : k) + pad, ldb = (TB ? k : n) + pad, ldc = n + pad;
  const std::int64_t arows = TA ? k : m, brows = TB ? n : k;
  const std::int64_t abytes = std::max<std::int64_t>(1, ((arows ? arows - 1 : 0) * lda + (TA ? m : k)) * ES);
  const std::int64_t bbytes = std::max<std::int64_t>(1, ((brows ? brows - 1 : 0) * ldb + (TB ? k : n)) * ES);
  std::vector<std::uint8_t> A(abytes, 0x7f), B(bbytes, 0x7f);
  for(std::int64_t r = 0; r < arows; ++r)
    for(int q = 0; q < (TA ? m : k); ++q) put<ES>(A, r * lda + q, mix(11 + r * 7919 + q));
  for(std::int64_t r = 0; r < brows; ++r)
    for(int q = 0; q < (TB ? k : n); ++q) put<ES>(B, r * ldb + q, mix(23 + r * 104729 + q));
  auto a_at = [&](int i, int p) { return TA ? std::int64_t(p) * lda + i : std::int64_t(i) * lda + p; };
  auto b_at = [&](int p, int j) { return TB ? std::int64_t(j) * ldb + p : std::int64_t(p) * ldb + j; };
  std::vector<double> C(std::size_t(m) * ldc), old(std::size_t(m) * ldc);
  std::vector<int> written(std::size_t(m) * ldc);
  for(std::size_t e = 0; e < C.size(); ++e) C[e] = old[e] = double(std::int64_t(mix(99 + e) % 9) - 4) / 4.0;

  const int tiles_m = (m + BM - 1) / BM, tiles_n = (n + BN - 1) / BN, total = tiles_m * tiles_n;
  HostMem mem_a{reinterpret_cast<const char*>(A.data()), reinterpret_cast<const char*>(A.data()) + A.size()};
  HostMem mem_b{reinterpret_cast<const char*>(B.data()), reinterpret_cast<const char*>(B.data()) + B.size()};
  for(int wg = 0; wg < total; ++wg) {
    int tm, tn;
    tile_of(wg, tiles_m, tiles_n, group, tm, tn);
    const int row0 = tm * BM, col0 = tn * BN;
    const Panel pa = panel(AK, row0, m, k, lda, ES), pb = panel(BKM, col0, n, k, ldb, ES);
    const char* a = reinterpret_cast<const char*>(A.data()) + pa.start;
    const char* b = reinterpret_cast<const char*>(B.data()) + pb.start;
    std::vector<cairn::pipe::Loader<Sh, BM, AK, HostDma>> la(256);
    std::vector<cairn::pipe::Loader<Sh, BN, BKM, HostDma>> lb(256);
    for(int gt = 0; gt < 256; ++gt) {
      la[gt].setup(gt, row0, m, lda);
      lb[gt].setup(gt, col0, n, ldb);
    }
    std::vector<double> acc(static_cast<std::size_t>(BM * BN), 0.0);
    const int T = (k + Sh::BK - 1) / Sh::BK;
    using LAx = cairn::pipe::Loader<Sh, BM, AK, HostDma>;
    using LBx = cairn::pipe::Loader<Sh, BN, BKM, HostDma>;
    for(int st = 0; st < T; ++st) {
      HostLds lds(Sh::STAGE);  // one stage of the ring (the ring's other stages are the same code at other bases)
      HostDma da{&mem_a, &lds, lds.bytes.data()}, db{&mem_b, &lds, lds.bytes.data()};
      using LA = cairn::pipe::Loader<Sh, BM, AK, HostDma>;
      using LB = cairn::pipe::Loader<Sh, BN, BKM, HostDma>;
      // The one-wave-a-SIMD kernel loads through M0 and immediate offsets where the leading dimensions allow it.
      const bool imm = Sh::WAVES == 4 && LA::imm_fits(lda) && LB::imm_fits(ldb);
      char* stage_a = reinterpret_cast<char*>(lds.bytes.data());
      char* stage_b = stage_a + Sh::A_BYTES;
      for(int gt = 0; gt < 256; ++gt) {
        da.lane = db.lane = gt & 63;
        if(imm && (st + 1) * Sh::BK <= k) {  // the main loop's steady loads, through the walked resources
          da.set_base(LA::base(stage_a, gt >> 6));
          steady_loads(la[gt], da, walked<Sh, AK>(mem_a, a, pa.bytes, lda, st), std::make_index_sequence<LA::LOADS>{});
          db.set_base(LB::base(stage_b, gt >> 6));
          steady_loads(lb[gt], db, walked<Sh, BKM>(mem_b, b, pb.bytes, ldb, st), std::make_index_sequence<LB::LOADS>{});
        } else if(imm) {
          da.set_base(LA::base(stage_a, gt >> 6));
          imm_loads(la[gt], da, la[gt].resource(da, a, pa.bytes, lda, st), st, k, std::make_index_sequence<LA::LOADS>{});
          db.set_base(LB::base(stage_b, gt >> 6));
          imm_loads(lb[gt], db, lb[gt].resource(db, b, pb.bytes, ldb, st), st, k, std::make_index_sequence<LB::LOADS>{});
        } else {
          la[gt].issue(da, a, pa.bytes, lda, st, k, stage_a, gt >> 6);
          lb[gt].issue(db, b, pb.bytes, ldb, st, k, stage_b, gt >> 6);
        }
      }
      if(da.negative || db.negative) FAIL("pipe %s %dx%d es=%d %dx%dx%d: an offset register below zero", lay, BM, BN, ES, m, n, k);
      if(mem_a.bad || mem_b.bad) FAIL("pipe %s %dx%d es=%d %dx%dx%d: a global load outside its matrix", lay, BM, BN, ES, m, n, k);
      if(lds.bad) FAIL("pipe %s: an LDS write off the stage", lay);
      for(int c = 0; c < Sh::STAGE / 16; ++c)
        if(lds.writes[c] != 1) FAIL("pipe %s %dx%d es=%d: LDS chunk %d written %d times", lay, BM, BN, ES, c, lds.writes[c]);
      for(int wave = 0; wave < Sh::WAVES; ++wave) {
        int wr, wc;
        cairn::pipe::wave_origin<Sh>(wave, wr, wc);
        for(int s = 0; s < 2; ++s)
          for(int i = 0; i < Sh::FM; ++i)
            for(int j = 0; j < Sh::FN; ++j) {
              std::uint8_t fa[64][16], fb[64][16];
              auto gather = [&](bool kmajor, int base, int R, int row0_, std::uint8_t (&out)[64][16]) {
                if(kmajor) {
                  int addr[64];
                  for(int l = 0; l < 64; ++l) {
                    const int at = base + cairn::pipe::kmajor_fragment(row0_, s, l);
                    addr[l] = at;
                    if(at < base || at + 16 > base + R * 64) bad_read = true;
                    std::memcpy(out[l], &lds.bytes[at], 16);
                  }
                  check_banks(addr, 16);
                } else {
                  for(int h = 0; h < 2; ++h) {
                    int addr[64];
                    for(int l = 0; l < 64; ++l) {
                      addr[l] = base + (R == BM ? frag_mn<ES, BM>(row0_, s, h, l) : frag_mn<ES, BN>(row0_, s, h, l));
                      if(addr[l] < base || addr[l] + 8 > base + R * 64) bad_read = true;
                      // The kernel's form: the lane's k-step 0, half 0 offset, then an immediate step.
                      const int stepped = R == BM ? frag_mn<ES, BM>(row0_, 0, 0, l) + cairn::pipe::mnmajor_step<ES, BM>(s, h)
                                                  : frag_mn<ES, BN>(row0_, 0, 0, l) + cairn::pipe::mnmajor_step<ES, BN>(s, h);
                      if(base + stepped != addr[l]) stepped_off = true;
                    }
                    check_banks(addr, 8);
                    std::uint8_t got[64][8];
                    cairn::pipe::transpose_read(lds.bytes.data(), addr, ES, got);
                    for(int l = 0; l < 64; ++l) std::memcpy(out[l] + 8 * h, got[l], 8);
                  }
                }
              };
              gather(AK, 0, BM, wr + 32 * i, fa);
              gather(BKM, Sh::A_BYTES, BN, wc + 32 * j, fb);
              if(bad_read) FAIL("pipe %s: a fragment read off its operand's stage", lay);
              if(stepped_off) FAIL("pipe %s %dx%d es=%d: a transpose read's k-step and half are not an immediate step", lay, BM, BN, ES);
              if(conflict) FAIL("pipe %s %dx%d es=%d: a fragment read phase has an LDS bank conflict", lay, BM, BN, ES);
              double P[32][32], Q[32][32];
              constexpr int CE = 16 / ES;
              for(int l = 0; l < 64; ++l) {
                double pv[16], qv[16];
                decode<ES>(fb[l], pv);
                decode<ES>(fa[l], qv);
                for(int e = 0; e < CE; ++e) {
                  P[l & 31][(l >> 5) * CE + e] = pv[e];
                  Q[(l >> 5) * CE + e][l & 31] = qv[e];
                }
              }
              for(int l = 0; l < 64; ++l)
                for(int r = 0; r < 16; ++r) {
                  const int prow = 8 * (r / 4) + 4 * (l / 32) + r % 4, qcol = l % 32;
                  double sum = 0;
                  for(int kk = 0; kk < 2 * CE; ++kk) sum += P[prow][kk] * Q[kk][qcol];
                  const int mm = wr + 32 * i + acc_m(l);
                  const int nn = wc + 32 * j + acc_n(l, r / 4) + r % 4;
                  acc[std::size_t(mm) * BN + nn] += sum;
                }
            }
      }
    }
    // Where k is a whole number of stages, the one-wave-a-SIMD kernel's main loop also issues steady loads for the S
    // stages past the last (into ring buffers no MFMA reads again): each must stay inside its matrix or read zeros.
    if(Sh::WAVES == 4 && k % Sh::BK == 0 && LAx::imm_fits(lda) && LBx::imm_fits(ldb)) {
      HostLds spare(Sh::STAGE);
      HostDma da{&mem_a, &spare, spare.bytes.data()}, db{&mem_b, &spare, spare.bytes.data()};
      char* stage_a = reinterpret_cast<char*>(spare.bytes.data());
      for(int st = T; st < T + Sh::STAGES; ++st)
        for(int gt = 0; gt < 256; ++gt) {
          da.lane = db.lane = gt & 63;
          da.set_base(LAx::base(stage_a, gt >> 6));
          steady_loads(la[gt], da, walked<Sh, AK>(mem_a, a, pa.bytes, lda, st), std::make_index_sequence<LAx::LOADS>{});
          db.set_base(LBx::base(stage_a + Sh::A_BYTES, gt >> 6));
          steady_loads(lb[gt], db, walked<Sh, BKM>(mem_b, b, pb.bytes, ldb, st), std::make_index_sequence<LBx::LOADS>{});
        }
      if(mem_a.bad || mem_b.bad) FAIL("pipe %s %dx%d es=%d %dx%dx%d: a load past the last stage outside its matrix", lay, BM, BN, ES, m, n, k);
      if(da.negative || db.negative) FAIL("pipe %s: an offset register below zero past the last stage", lay);
    }
    for(int wave = 0; wave < Sh::WAVES; ++wave) {
      int wr, wc;
      cairn::pipe::wave_origin<Sh>(wave, wr, wc);
      for(int i = 0; i < Sh::FM; ++i)
        for(int j = 0; j < Sh::FN; ++j)
          for(int l = 0; l < 64; ++l)
            for(int q = 0; q < 4; ++q) {
              const int mm = wr + 32 * i + acc_m(l), nn0 = wc + 32 * j + acc_n(l, q);
              const int gm = row0 + mm, gn = col0 + nn0;
              if(gm >= m || gn >= n) continue;
              for(int e = 0; e < 4; ++e) {
                const std::size_t at = std::size_t(gm) * ldc + gn + e;
                C[at] = old[at] + acc[std::size_t(mm) * BN + nn0 + e];
                ++written[at];
              }
            }
    }
  }
  for(int i = 0; i < m; ++i)
    for(int j = 0; j < n; ++j) {
      double exact = 0;
      for(int p = 0; p < k; ++p) exact += value_of<ES>(A, a_at(i, p)) * value_of<ES>(B, b_at(p, j));
      const std::size_t at = std::size_t(i) * ldc + j;
      if(written[at] != 1) FAIL("pipe %s %dx%d es=%d %dx%dx%d: output (%d,%d) written %d times", lay, BM, BN, ES, m, n, k, i, j, written[at]);
      if(C[at] != old[at] + exact)
        FAIL("pipe %s %dx%d es=%d %dx%dx%d pad %d: output (%d,%d) is %.9g, exact %.9g", lay, BM, BN, ES, m, n, k, pad, i,
             j, C[at], old[at] + exact);
    }
}

template<class Sh> void pipe_shapes() {
  constexpr int CE = 16 / Sh::ES, MN = Sh::ES == 2 ? 8 : 16;  // k chunk; m, n pieces of an M/N-major row
  const int list[][5] = {{MN, MN, CE, 0, 4},
                         {Sh::BM, Sh::BN, 64 / Sh::ES, 0, 4},
                         {Sh::BM + MN, Sh::BN + 2 * MN, 3 * CE, 16, 1},
                         {2 * Sh::BM + 4 * MN, Sh::BN - MN, 200 / CE * CE, 16, 2},
                         {264 / MN * MN, Sh::BN + MN, 37 * CE, 0, 4},
                         {Sh::BM + MN, Sh::BN, 8 * (64 / Sh::ES), 8, 3}};
  for(auto& s : list) {
    run_pipe<Sh, false, false>(s[0], s[1], s[2], s[3], s[4]);
    run_pipe<Sh, false, true>(s[0], s[1], s[2], s[3], s[4]);
    run_pipe<Sh, true, false>(s[0], s[1], s[2], s[3], s[4]);
    run_pipe<Sh, true, true>(s[0], s[1], s[2], s[3], s[4]);
  }
}

template<int BM, int BN, int ES, int W> void layouts(int m, int n, int k, int pad, int group) {
  run<BM, BN, ES, false, false, W>(m, n, k, pad, group);
  run<BM, BN, ES, false, true, W>(m, n, k, pad, group);
  run<BM, BN, ES, true, false, W>(m, n, k, pad, group);
  run<BM, BN, ES, true, true, W>(m, n, k, pad, group);
}

template<int BM, int BN, int ES, int W = WIDEN_NONE> void shapes() {
  // m and n multiples of 8 (the MN-major fetch's 8-column pieces), k a multiple of the 16-byte LDS chunk; tails in
  // every direction against the tile and the k-step, padded (by 8: the widened 8-bit floats' 8-byte pieces) and
  // packed leading dimensions, one and several groups.
  constexpr int CE = 16 / ES;
  const int list[][5] = {{8, 8, CE, 0, 4},           {64, 64, 4 * CE, 8, 4},      {BM, BN, 128 / ES, 0, 4},
                         {BM + 8, BN + 24, 3 * CE, 8, 1}, {2 * BM + 72, BN - 8, 200 / CE * CE, 16, 2},
                         {264, 3 * BN + 8, 19 * CE, 0, 4}};
  for(auto& s : list) layouts<BM, BN, ES, W>(s[0], s[1], s[2], s[3], s[4]);
}

}  // namespace

int main() {
  pipe_shapes<cairn::pipe::Shape<256, 256, 2, 4>>();
  pipe_shapes<cairn::pipe::Shape<256, 256, 1, 4>>();
  pipe_shapes<cairn::pipe::Shape<256, 128, 2, 4>>();
  pipe_shapes<cairn::pipe::Shape<128, 256, 2, 4>>();
  pipe_shapes<cairn::pipe::Shape<128, 128, 2, 4>>();
  pipe_shapes<cairn::pipe::Shape<128, 128, 1, 4>>();
  pipe_shapes<cairn::pipe::Shape<256, 256, 2, 4, 4>>();
  pipe_shapes<cairn::pipe::Shape<256, 256, 1, 4, 4>>();
  pipe_shapes<cairn::pipe::Shape<256, 256, 2, 5, 4>>();  // a 5-stage ring (the index math is the same)
  pipe_shapes<cairn::pipe::Shape<256, 128, 2, 4, 4>>();
  pipe_shapes<cairn::pipe::Shape<128, 128, 2, 4, 4>>();
  pipe_shapes<cairn::pipe::Shape<128, 128, 1, 4, 4>>();
  if(failures) {
    std::printf("pipe: %d failures\n", failures);
    return 1;
  }
  shapes<256, 256, 2>();
  shapes<256, 128, 2>();
  shapes<128, 256, 2>();
  shapes<128, 128, 2>();
  shapes<256, 256, 1>();
  shapes<256, 128, 1>();
  shapes<128, 128, 1>();
  widening_is_exact();
  shapes<128, 128, 2, WIDEN_E4M3>();
  shapes<128, 128, 2, WIDEN_E5M2>();
  // tile_of is a bijection for grids whose size is and is not a multiple of 8, and for partial groups.
  for(int tm = 1; tm <= 13; ++tm)
    for(int tn = 1; tn <= 11; ++tn)
      for(int g = 1; g <= 5; ++g) {
        std::vector<int> seen(tm * tn);
        for(int b = 0; b < tm * tn; ++b) {
          int x, y;
          tile_of(b, tm, tn, g, x, y);
          if(x < 0 || x >= tm || y < 0 || y >= tn) {
            std::printf("tile_of off the grid\n");
            return 1;
          }
          ++seen[x * tn + y];
        }
        for(int v : seen)
          if(v != 1) {
            std::printf("tile_of is not a bijection at %d x %d group %d\n", tm, tn, g);
            return 1;
          }
      }
  // The split last round, per XCD block: every (tile, stage) in exactly one unit's segment, every slot used once over
  // all XCDs, each tile's units (split_units_of) naming its segments in k order with the slots they were written to
  // (split_slot), and the whole-tile pass and the split tiles together covering every id once.
  for(int xcds : {1, 8})
    for(int tiles = 1; tiles <= 31; tiles += (tiles < 16 ? 1 : 5))
      for(int stages : {1, 2, 3, 4, 7, 16, 64, 65, 128})
        for(int units : {1, 7, 16, 31, 32}) {
          const long long total = (long long)tiles * stages;
          const int quota = int((total + units - 1) / units);
          if(quota > stages) continue;  // the planner never asks for this
          const int first = 64, block = first + tiles;
          Split s{first, tiles, stages, quota, int((total + quota - 1) / quota), xcds, block};
          std::vector<int> slot_used(2 * xcds * s.units, 0), id_seen(xcds * block, 0);
          for(int b = 0; b < xcds * first; ++b) ++id_seen[whole_id(s, b)];
          for(int x = 0; x < xcds; ++x) {
            std::vector<int> owner(total, -1);
            for(int v = 0; v < s.units; ++v)
              for(int j = 0; j < 2; ++j) {
                int tile, s0, s1;
                if(!split_segment(s, v, j, tile, s0, s1)) continue;
                const int slot = 2 * (v * xcds + x) + j;  // what workgroup u = v xcds + x writes
                if(tile < 0 || tile >= tiles || s0 < 0 || s1 > stages || s0 >= s1 || slot_used[slot]++) {
                  std::printf("split segment off its tile, or a slot written twice\n");
                  return 1;
                }
                for(int st = s0; st < s1; ++st) {
                  if(owner[(long long)tile * stages + st] != -1) {
                    std::printf("split stage run twice\n");
                    return 1;
                  }
                  owner[(long long)tile * stages + st] = slot;
                }
              }
            for(int o : owner)
              if(o < 0) {
                std::printf("split stage never run (%d tiles, %d stages, %d units)\n", tiles, stages, units);
                return 1;
              }
            for(int tl = 0; tl < tiles; ++tl) {
              ++id_seen[split_id(s, x, tl)];
              int lo, hi;
              split_units_of(s, tl, lo, hi);
              int next = 0;  // the tile's next stage in k order
              for(int v = lo; v <= hi; ++v) {
                const int slot = split_slot(s, x, tl, v);
                if(owner[(long long)tl * stages + next] != slot) {
                  std::printf("split fixup reads the wrong slot\n");
                  return 1;
                }
                while(next < stages && owner[(long long)tl * stages + next] == slot) ++next;
              }
              if(next != stages) {
                std::printf("split fixup misses stages of a tile\n");
                return 1;
              }
            }
          }
          for(int seen : id_seen)
            if(seen != 1) {
              std::printf("the two passes do not cover every tile id once\n");
              return 1;
            }
        }
  if(failures) return 1;
  std::printf("ok: every tile equals the exact product\n");
  return 0;
}
