// The C ABI of libcairn_gemm_gfx950.so (include/cairn_gemm.h): the kernel table, the checks a descriptor must pass,
// the tile selector and the launch. No allocation, no stream or event made, no wait: cairn_gemm_run only queues.
#include <hip/hip_runtime.h>
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstddef>
#include <cstring>
#include <initializer_list>
#include "../../include/cairn_gemm.h"
#include "kernels.hpp"

using cairn::gemm::Params;
using Launcher = hipError_t (*)(const Params&, hipStream_t);

#define CAIRN_MFMA_INSTANCE(NAME, BM, BN, OP, TA, TB) hipError_t NAME(const Params&, hipStream_t);
#include "instances.inc"
#undef CAIRN_MFMA_INSTANCE
#define CAIRN_WAVE_INSTANCE(NAME, BM, BN, STAGES, OP, TA, TB) hipError_t NAME(const Params&, hipStream_t);
#define CAIRN_WAVE8_INSTANCE(NAME, BM, BN, STAGES, OP, TA, TB) hipError_t NAME(const Params&, hipStream_t);
#include "wave_instances.inc"
#undef CAIRN_WAVE_INSTANCE
#undef CAIRN_WAVE8_INSTANCE
hipError_t cairn_generic(const Params&, hipStream_t);
hipError_t cairn_skinny(const Params&, hipStream_t, int split);
int cairn_skinny_width(int n);

namespace {

constexpr int CUS = 256;              // gfx950: 8 XCDs of 32 CUs (MI350X, MI355X)
constexpr int XCDS = 8;
constexpr int LDS_PER_CU = 160 * 1024;

enum Family { MFMA = 0, GENERIC = 1, SKINNY = 2, WAVE = 4 };  // 3 was an eight-wave kernel, retired

struct Kernel {
  Launcher run;
  int family;
  int op;  // cairn::gemm::OP_*; the generic and skinny kernels take every type they are given
  bool ta, tb;
  int bm, bn;
  const char* name;
  int stages;  // LDS stages (the tiled kernels)
};

#define CAIRN_MFMA_INSTANCE(NAME, BM, BN, OP, TA, TB) {NAME, MFMA, OP, TA, TB, BM, BN, #NAME, 2},
#define CAIRN_WAVE_INSTANCE(NAME, BM, BN, STAGES, OP, TA, TB) {NAME, WAVE, OP, TA, TB, BM, BN, #NAME, STAGES},
#define CAIRN_WAVE8_INSTANCE(NAME, BM, BN, STAGES, OP, TA, TB) {NAME, WAVE, OP, TA, TB, BM, BN, #NAME, STAGES},
const Kernel TABLE[] = {
    {nullptr, GENERIC, -1, false, false, 64, 64, "cairn_generic_64x64", 1},
    {nullptr, SKINNY, cairn::gemm::OP_BF16, false, true, 16, 64, "cairn_skinny_bf16_nt", 0},
#include "instances.inc"
#include "wave_instances.inc"
};
#undef CAIRN_MFMA_INSTANCE
#undef CAIRN_WAVE_INSTANCE
#undef CAIRN_WAVE8_INSTANCE
constexpr int COUNT = int(sizeof(TABLE) / sizeof(TABLE[0]));

int op_of(int type) {
  switch(type) {
    case CAIRN_TYPE_BF16: return cairn::gemm::OP_BF16;
    case CAIRN_TYPE_F16: return cairn::gemm::OP_F16;
    case CAIRN_TYPE_I8: return cairn::gemm::OP_I8;
    case CAIRN_TYPE_F8E4M3: return cairn::gemm::OP_F8E4M3;  // the MFMA and generic kernels widen them to f16; the
    case CAIRN_TYPE_F8E5M2: return cairn::gemm::OP_F8E5M2;  // ring's wave8 form runs the 8-bit float matrix core
    default: return -1;
  }
}
int element_size(int type) { return type == CAIRN_TYPE_BF16 || type == CAIRN_TYPE_F16 ? 2 : 1; }
int output_size(int type) { return type == CAIRN_TYPE_F32 || type == CAIRN_TYPE_I32 ? 4 : 2; }
bool aligned(const void* p, std::uint64_t bytes) { return reinterpret_cast<std::uintptr_t>(p) % bytes == 0; }

// A descriptor with its leading dimensions filled in, checked.
struct Problem {
  cairn_gemm_desc d;
  bool empty;  // nothing to queue
};

int check(const cairn_gemm_desc* in, Problem& out) {
  if(!in || (in->version != 1u && in->version != CAIRN_GEMM_DESC_VERSION)) return CAIRN_E_ARG;
  // A version 1 descriptor ends at `kernel`: the fields after it are not read, and it never splits.
  cairn_gemm_desc d{};
  std::memcpy(&d, in, in->version == 1u ? offsetof(cairn_gemm_desc, workspace) : sizeof(d));
  if(in->version == 1u) d.split_units = -1;
  if(d.split_units < -1 || (d.workspace && reinterpret_cast<std::uintptr_t>(d.workspace) % 256)) return CAIRN_E_ARG;
  const int t = d.ab_type;
  if(t != CAIRN_TYPE_F16 && t != CAIRN_TYPE_BF16 && t != CAIRN_TYPE_F8E4M3 && t != CAIRN_TYPE_F8E5M2 &&
     t != CAIRN_TYPE_I8)
    return CAIRN_E_TYPE;
  const bool epilogue = d.bias || d.row_scale || d.col_scale || d.act != CAIRN_ACT_NONE;
  if(d.c_type == CAIRN_TYPE_I32) {
    if(t != CAIRN_TYPE_I8 || epilogue || d.accumulate) return CAIRN_E_TYPE;  // the accumulator itself
  } else if(d.c_type != CAIRN_TYPE_F32 && d.c_type != CAIRN_TYPE_BF16 && d.c_type != CAIRN_TYPE_F16) {
    return CAIRN_E_TYPE;
  }
  if(d.accumulate && d.c_type != CAIRN_TYPE_F32) return CAIRN_E_TYPE;
  if(d.act < CAIRN_ACT_NONE || d.act > CAIRN_ACT_GELU) return CAIRN_E_ARG;
  if(d.bias && d.bias_type != CAIRN_TYPE_F32 && d.bias_type != CAIRN_TYPE_BF16) return CAIRN_E_TYPE;
  if((d.trans_a != 0 && d.trans_a != 1) || (d.trans_b != 0 && d.trans_b != 1)) return CAIRN_E_ARG;
  // Extents leave room below 2^31 for the largest tile: the kernels compare row0 + BM (col0 + BN, k0 + BK) with an
  // extent in 32-bit arithmetic, which must not wrap for the last tile.
  constexpr std::uint64_t LIMIT = 0x7fffffffULL, EXTENT = 0x7fffff00ULL;
  if(d.m > EXTENT || d.n > EXTENT || d.k > EXTENT) return CAIRN_E_SHAPE;
  const std::uint64_t arow = d.trans_a ? d.m : d.k, brow = d.trans_b ? d.k : d.n;
  if(!d.lda) d.lda = arow;
  if(!d.ldb) d.ldb = brow;
  if(!d.ldc) d.ldc = d.n;
  if(d.lda < arow || d.ldb < brow || d.ldc < d.n) return CAIRN_E_SHAPE;
  out.empty = d.m == 0 || d.n == 0 || (d.k == 0 && d.c_type == CAIRN_TYPE_F32 && d.accumulate && !epilogue);
  if(!out.empty) {
    if(!d.c) return CAIRN_E_ARG;
    if(d.k && (!d.a || !d.b)) return CAIRN_E_ARG;
    // Workgroup counts and element offsets fit the kernels' int32 and 64-bit arithmetic.
    if(((d.m + 63) / 64) * ((d.n + 63) / 64) > LIMIT) return CAIRN_E_SHAPE;
  }
  out.d = d;
  return CAIRN_OK;
}

// Is d's operand type an 8-bit float (which the MFMA kernel widens to f16 on its way into LDS).
bool float8(int type) { return type == CAIRN_TYPE_F8E4M3 || type == CAIRN_TYPE_F8E5M2; }

// Can the tiled MFMA kernel take this problem: its 16-byte LDS chunks whole and aligned in memory (8 bytes of the
// 8-bit floats, which widen to 16), its offsets inside int32.
bool mfma_fits(const cairn_gemm_desc& d, const Kernel& k) {
  if(k.family != MFMA || k.op != op_of(d.ab_type) || k.ta != bool(d.trans_a) || k.tb != bool(d.trans_b)) return false;
  const int gs = element_size(d.ab_type), es = float8(d.ab_type) ? 2 : gs, ce = 16 / es;
  const std::uint64_t bk = 128 / es;
  auto kmajor = [&](const void* p, std::uint64_t ld, int rows) {
    return d.k % ce == 0 && ld % ce == 0 && aligned(p, ce * gs) && std::uint64_t(rows) * ld * gs < 0x7fff0000ULL;
  };
  auto mnmajor = [&](const void* p, std::uint64_t ld, std::uint64_t cols) {
    return cols % 8 == 0 && ld % 8 == 0 && aligned(p, 8 * gs) && bk * ld * gs < 0x7fff0000ULL;
  };
  const bool a_ok = d.trans_a ? mnmajor(d.a, d.lda, d.m) : kmajor(d.a, d.lda, k.bm);
  const bool b_ok = d.trans_b ? kmajor(d.b, d.ldb, k.bn) : mnmajor(d.b, d.ldb, d.n);
  const int os = output_size(d.c_type);
  const bool c_ok = d.n % 4 == 0 && d.ldc % 4 == 0 && aligned(d.c, 4 * os);
  return a_ok && b_ok && c_ok;
}

// Can a kernel of the LDS ring (one wave a SIMD) take it: 16-byte loads whole and aligned (K-major rows
// in chunks of 16 bytes of k; M/N-major rows in chunks of 16 bytes of columns), offsets inside int32.
bool ring(const Kernel& k) { return k.family == WAVE; }
bool ring_fits(const cairn_gemm_desc& d, const Kernel& k) {
  if(!ring(k) || k.op != op_of(d.ab_type) || k.ta != bool(d.trans_a) || k.tb != bool(d.trans_b)) return false;
  const int es = element_size(d.ab_type), ce = 16 / es;
  const std::uint64_t bk = 64 / es;
  auto kmajor = [&](const void* p, std::uint64_t ld, int rows) {
    return d.k % ce == 0 && ld % ce == 0 && aligned(p, 16) && std::uint64_t(rows) * ld * es < 0x7fff0000ULL;
  };
  auto mnmajor = [&](const void* p, std::uint64_t ld, std::uint64_t cols) {
    return cols % ce == 0 && ld % ce == 0 && aligned(p, 16) && bk * ld * es < 0x7fff0000ULL;
  };
  const bool a_ok = d.trans_a ? mnmajor(d.a, d.lda, d.m) : kmajor(d.a, d.lda, k.bm);
  const bool b_ok = d.trans_b ? kmajor(d.b, d.ldb, k.bn) : mnmajor(d.b, d.ldb, d.n);
  const int os = output_size(d.c_type);
  const bool c_ok = d.n % 4 == 0 && d.ldc % 4 == 0 && aligned(d.c, 4 * os);
  // The one-wave-a-SIMD kernel loads by immediate offsets (pipe.hpp, Loader::imm_fits): a K-major operand's rows at
  // least a stage's 64 bytes apart, an M/N-major operand's k rows at least a tile's width of elements apart.
  auto imm = [&](bool kmaj, std::uint64_t ld, int width) { return kmaj ? ld * es >= 64 : ld >= std::uint64_t(width); };
  const bool imm_ok = (imm(!d.trans_a, d.lda, k.bm) && imm(bool(d.trans_b), d.ldb, k.bn));
  return a_ok && b_ok && c_ok && imm_ok;
}

bool tiled_fits(const cairn_gemm_desc& d, const Kernel& k) { return ring(k) ? ring_fits(d, k) : mfma_fits(d, k); }

// The skinny kernel: bf16, b stored n x k (the decode layout), m <= 16, every row 16-byte whole.
bool skinny_fits(const cairn_gemm_desc& d) {
  return d.ab_type == CAIRN_TYPE_BF16 && !d.trans_a && d.trans_b && d.m <= 16 && d.k % 8 == 0 && d.lda % 8 == 0 &&
         d.ldb % 8 == 0 && aligned(d.a, 16) && aligned(d.b, 16) && d.lda * 2 * 16 < 0x7fff0000ULL &&
         d.ldb * 2 * 64 < 0x7fff0000ULL;
}

// Workgroups of a tile shape one CU holds at once: LDS is the limit (two stages of both operands).
int lds_bytes(const Kernel& k) {
  if(ring(k)) return k.stages * (k.bm + k.bn) * 64;
  if(k.family == MFMA) return 2 * (k.bm + k.bn) * 128;
  return k.family == GENERIC ? 4096 : 16384;  // skinny: four waves' partial sums
}
int resident(const Kernel& k) {
  if(k.family != MFMA && !ring(k)) return 8;
  const int lds = lds_bytes(k);
  return std::max(1, std::min(2, LDS_PER_CU / lds));
}

// k elements a k-step of the kernel covers.
int tile_k(const Kernel& k) {
  const int bytes = k.family == MFMA ? 128 : (ring(k) ? 64 : 32);
  if(k.family == SKINNY) return 32;
  const bool f8 = k.op == cairn::gemm::OP_F8E4M3 || k.op == cairn::gemm::OP_F8E5M2;
  const bool byte = k.op == cairn::gemm::OP_I8 || (f8 && k.family != MFMA);  // the MFMA kernel holds them as f16
  return byte ? bytes : bytes / 2;
}

// The split last round a ring kernel would run for d with `room` workspace bytes (cairn::tile::Split). The tile ids
// are dealt to the 8 XCDs in blocks (where the tile count divides into 8 blocks; else one block); each block keeps
// whole rounds of its XCD's CUs for the whole-tile pass and splits the rest. No split where the blocks are whole
// rounds, a split is not asked for or would not pay (below), or the room holds too few units; the selector's choice takes a unit a CU, as many as the room holds, and no unit with
// fewer than SPLIT_MIN stages (a segment pays its own prologue and a partial tile's stores). A split asked for
// explicitly (split_units > 0, for the whole machine) that cannot run is refused instead.
struct Plan {
  std::uint64_t whole;  // workgroups of the whole-tile pass
  cairn::tile::Split split;
  std::uint64_t bytes;  // workspace the split uses
  int status;
};
Plan plan_of(const cairn_gemm_desc& d, const Kernel& k, std::uint64_t room) {
  const std::uint64_t tiles = ((d.m + k.bm - 1) / k.bm) * ((d.n + k.bn - 1) / k.bn);
  const int xcds = tiles % XCDS == 0 ? XCDS : 1;
  const std::uint64_t block = tiles / xcds, per = CUS / xcds;  // ids and CUs an XCD block has
  Plan pl{tiles, {}, 0, CAIRN_OK};
  pl.split.first = int(block);
  pl.split.xcds = xcds;
  pl.split.block = int(block);
  const bool asked = d.split_units > 0;
  if(!ring(k) || d.split_units < 0 || d.k == 0) return pl;
  const std::uint64_t first = block / per * per, left = block - first;
  const std::uint64_t stages = (d.k + tile_k(k) - 1) / tile_k(k), slot = std::uint64_t(k.bm) * k.bn * 4;
  if(!left) return pl;
  constexpr std::uint64_t SPLIT_MIN = 8;
  const std::uint64_t units = asked ? std::max<std::uint64_t>(1, std::uint64_t(d.split_units) / xcds)
                                    : std::min({per, room / (2 * slot * xcds), (left * stages) / SPLIT_MIN});
  if(!units) return pl;
  const std::uint64_t quota = (left * stages + units - 1) / units;
  if(quota > stages) {  // a unit would reach into a third tile
    if(asked) pl.status = CAIRN_E_ARG;
    return pl;
  }
  // The selector splits only a last round that would keep at most a quarter of the XCD's CUs busy, over at least 16
  // stages. Measured on the MLP layer's shapes (5.375 and 2.69 rounds), a split round was slower than the whole one:
  // CUs left idle let the power-limited clock rise, so a partial round costs far less than a full one (96 of 256
  // tiles: 0.57 of a full round's time), while split units each fetch their own panels, with no reuse across tiles
  // in L2, and write partial tiles the fixup reads back.
  if(!asked && (stages < 16 || 4 * left > per || 4 * quota > 3 * stages)) return pl;
  const std::uint64_t used = (left * stages + quota - 1) / quota;  // units an XCD runs
  const std::uint64_t bytes = 2 * xcds * used * slot;
  if(bytes > room) {
    if(asked) pl.status = CAIRN_E_SCRATCH;
    return pl;
  }
  pl.whole = xcds * first;
  pl.split = cairn::tile::Split{int(first), int(left), int(stages), int(quota), int(used), xcds, int(block)};
  pl.bytes = bytes;
  return pl;
}
std::uint64_t room_of(const cairn_gemm_desc& d) { return d.workspace ? d.workspace_bytes : 0; }

struct Estimate {
  double waves, efficiency;
  std::uint64_t workgroups;
};

Estimate estimate(const cairn_gemm_desc& d, const Kernel& k, const Plan& plan) {
  Estimate e{};
  if(k.family == SKINNY) {
    const std::uint64_t width = std::uint64_t(cairn_skinny_width(int(d.n)));
    const std::uint64_t blocks = (d.n + width - 1) / width;
    e.workgroups = blocks;
    e.waves = double(blocks) / CUS;  // one workgroup of four waves a CU
    e.efficiency = 1.0;
    return e;
  }
  const std::uint64_t tm = (d.m + k.bm - 1) / k.bm, tn = (d.n + k.bn - 1) / k.bn;
  const std::uint64_t tiles = tm * tn, slots = std::uint64_t(CUS) * resident(k);
  // A split last round costs a unit's share of a tile's stages instead of a whole round.
  const double rounds = plan.split.tiles ? double(plan.whole / slots) + double(plan.split.quota) / plan.split.stages
                                         : std::ceil(double(tiles) / double(slots));
  e.workgroups = plan.split.tiles ? plan.whole + std::uint64_t(plan.split.xcds) * plan.split.units : tiles;
  e.waves = double(tiles) / double(slots);
  const double useful = double(d.m) * double(d.n);
  e.efficiency = useful / (rounds * double(slots) * double(k.bm) * double(k.bn));
  return e;
}

// The kernel for a checked problem: the named one if it can run it; else the ring kernel (256 x 256, one wave a SIMD)
// where its loads fit; else the 128 x 128 MFMA kernel where its chunks fit; else the skinny kernel for a decode-shaped
// bf16 problem (ahead of both, from m <= 16); else the generic kernel. There is one kernel of each family for a type
// and layout, so this is a ranking of families, and it is measured, not modelled (`bench.py --only selector`: NN, m
// and n from 256 to 4096, k = 1024 and 4096, bf16 and int8). The ring kernel was faster at every bf16 shape,
// including those where its fewer, larger tiles leave most CUs idle: a round of tiles takes about one tile's time
// however few tiles it holds (idle CUs let the power-limited clock rise), and a lone 256 x 256 tile finishes sooner
// than a lone 128 x 128 one. int8 is the exception: at k = 1024, wherever the MFMA kernel's tiles fit one to a CU
// (24 of the 36 int8 shapes at that k), it was faster, 15.7-18.8 us against 17.8-20.3 (int8's stages are half as
// many, so the larger tile's longer prologue and epilogue weigh more); past one tile a CU, and at k = 4096, it was not.
int choose(const cairn_gemm_desc& d, int named) {
  if(named) {
    if(named < 1 || named > COUNT) return -CAIRN_E_KERNEL;
    const Kernel& k = TABLE[named - 1];
    if(k.family == GENERIC) return named;
    if(k.family == SKINNY) return skinny_fits(d) && d.c_type != CAIRN_TYPE_I32 ? named : -CAIRN_E_KERNEL;
    return tiled_fits(d, k) ? named : -CAIRN_E_KERNEL;
  }
  if(d.m <= 16 && skinny_fits(d)) {
    for(int id = 1; id <= COUNT; ++id)
      if(TABLE[id - 1].family == SKINNY) return id;
  }
  const std::uint64_t small_tiles = ((d.m + 127) / 128) * ((d.n + 127) / 128);
  const bool short_i8 = d.ab_type == CAIRN_TYPE_I8 && d.k > 0 && d.k <= 1024 && small_tiles <= std::uint64_t(CUS);
  // The 8-bit floats go to the MFMA kernel, which widens them to f16: the ring's 8-bit float matrix core adds its
  // products with a narrower alignment than the contract allows (it runs only where named).
  const auto order = float8(d.ab_type) ? std::initializer_list<int>{MFMA}
                                       : (short_i8 ? std::initializer_list<int>{MFMA, WAVE}
                                                   : std::initializer_list<int>{WAVE, MFMA});
  for(const int family : order)
    for(int id = 1; id <= COUNT; ++id)
      if(TABLE[id - 1].family == family && tiled_fits(d, TABLE[id - 1])) return id;
  for(int id = 1; id <= COUNT; ++id)
    if(TABLE[id - 1].family == GENERIC) return id;
  return -CAIRN_E_KERNEL;
}

Params params_of(const cairn_gemm_desc& d, const Kernel& k, const Plan& plan) {
  Params p{};
  p.whole_tiles = int(plan.whole);
  p.split = plan.split;
  p.work = d.workspace;
  p.a = d.a;
  p.b = d.b;
  p.c = d.c;
  p.lda = std::int64_t(d.lda);
  p.ldb = std::int64_t(d.ldb);
  p.ldc = std::int64_t(d.ldc);
  p.m = int(d.m);
  p.n = int(d.n);
  p.k = int(d.k);
  p.tiles_m = int((d.m + k.bm - 1) / k.bm);
  p.tiles_n = int((d.n + k.bn - 1) / k.bn);
  p.group = 4;
  p.trans_a = d.trans_a;
  p.trans_b = d.trans_b;
  p.a_type = d.ab_type;
  p.c_type = d.c_type;
  p.accumulate = d.accumulate;
  p.act = d.act;
  p.bias = d.bias;
  p.bias_type = d.bias_type;
  p.row_scale = d.row_scale;
  p.col_scale = d.col_scale;
  p.rows16 = aligned(d.c, 16) && (d.ldc * std::uint64_t(output_size(d.c_type))) % 16 == 0;
  return p;
}

}  // namespace

extern "C" {

// The interface identity the header derives from its stated interface (CAIRN_GEMM_IDENTITY), naming the library.
__attribute__((visibility("default"))) const char CAIRN_GEMM_IDENTITY[] = "gemm_gfx950";

int cairn_gemm_kernel_count(void) { return COUNT; }

int cairn_gemm_kernel_info(int32_t id, cairn_gemm_kernel* out) {
  if(id < 1 || id > COUNT || !out) return CAIRN_E_KERNEL;
  const Kernel& k = TABLE[id - 1];
  std::memset(out, 0, sizeof(*out));
  out->id = id;
  out->ab_type = k.op == cairn::gemm::OP_BF16     ? CAIRN_TYPE_BF16
                 : k.op == cairn::gemm::OP_F16    ? CAIRN_TYPE_F16
                 : k.op == cairn::gemm::OP_I8     ? CAIRN_TYPE_I8
                 : k.op == cairn::gemm::OP_F8E4M3 ? CAIRN_TYPE_F8E4M3
                 : k.op == cairn::gemm::OP_F8E5M2 ? CAIRN_TYPE_F8E5M2
                                                  : -1;
  out->trans_a = k.ta;
  out->trans_b = k.tb;
  out->tile_m = k.bm;
  out->tile_n = k.bn;
  out->tile_k = tile_k(k);
  out->threads = 256;
  out->lds_bytes = lds_bytes(k);
  out->family = k.family;
  std::strncpy(out->name, k.name, sizeof(out->name) - 1);
  return CAIRN_OK;
}

const char* cairn_gemm_status_string(int status) {
  switch(status) {
    case CAIRN_OK: return "ok";
    case CAIRN_E_SHAPE: return "an extent or leading dimension is out of range";
    case CAIRN_E_TYPE: return "no kernel computes this combination of operand, output and bias types";
    case CAIRN_E_KERNEL: return "the kernel named cannot run this problem";
    case CAIRN_E_ARG: return "a required pointer is null or the descriptor is malformed";
    case CAIRN_E_HIP: return "the HIP runtime refused the launch";
    case CAIRN_E_SCRATCH: return "the split last round asked for needs more scratch than the workspace holds";
    default: return "unknown status";
  }
}

int cairn_gemm_select(const cairn_gemm_desc* desc, cairn_gemm_choice* out) {
  Problem pr;
  if(const int s = check(desc, pr)) return s;
  const int id = choose(pr.d, desc->kernel);
  if(id < 0) return -id;
  const Kernel& k = TABLE[id - 1];
  const Plan plan = plan_of(pr.d, k, room_of(pr.d));
  if(plan.status) return plan.status;
  if(out) {
    const Estimate e = estimate(pr.d, k, plan);
    std::memset(out, 0, sizeof(*out));
    out->split_tiles = plan.split.xcds * plan.split.tiles;
    out->split_units = plan.split.xcds * plan.split.units;
    out->split_bytes = plan.bytes;
    out->kernel = id;
    out->family = k.family;
    out->tile_m = k.bm;
    out->tile_n = k.bn;
    out->tile_k = tile_k(k);
    out->workgroups = e.workgroups;
    out->waves = e.waves;
    out->efficiency = e.efficiency;
  }
  return CAIRN_OK;
}

int cairn_gemm_workspace(const cairn_gemm_desc* desc, uint64_t* bytes) {
  Problem pr;
  if(const int s = check(desc, pr)) return s;
  const int id = choose(pr.d, desc->kernel);
  if(id < 0) return -id;
  const Plan plan = plan_of(pr.d, TABLE[id - 1], ~std::uint64_t(0));
  if(plan.status) return plan.status;
  if(bytes) *bytes = pr.empty ? 0 : plan.bytes;
  return CAIRN_OK;
}

int cairn_gemm_run(const cairn_gemm_desc* desc, void* stream) {
  Problem pr;
  if(const int s = check(desc, pr)) return s;
  const int id = choose(pr.d, desc->kernel);
  if(id < 0) return -id;
  if(pr.empty) return CAIRN_OK;
  const Kernel& k = TABLE[id - 1];
  const Plan plan = plan_of(pr.d, k, room_of(pr.d));
  if(plan.status) return plan.status;
  const Params p = params_of(pr.d, k, plan);
  const hipStream_t s = static_cast<hipStream_t>(stream);
  hipError_t e;
  if(k.family == GENERIC) e = cairn_generic(p, s);
  else if(k.family == SKINNY) e = cairn_skinny(p, s, 0);
  else e = k.run(p, s);
  return e == hipSuccess ? CAIRN_OK : CAIRN_E_HIP;
}

int cairn_gemm_mma(int32_t type, size_t m, size_t n, size_t k, float* c, const void* a, const void* b,
                   void* stream) {
  if(type != CAIRN_TYPE_F16 && type != CAIRN_TYPE_BF16 && type != CAIRN_TYPE_F8E4M3 && type != CAIRN_TYPE_F8E5M2)
    return CAIRN_E_TYPE;
  cairn_gemm_desc d{};
  d.version = CAIRN_GEMM_DESC_VERSION;
  d.ab_type = type;
  d.c_type = CAIRN_TYPE_F32;
  d.m = m;
  d.n = n;
  d.k = k;
  d.a = a;
  d.b = b;
  d.c = c;
  d.accumulate = 1;
  return cairn_gemm_run(&d, stream);
}

}  // extern "C"
