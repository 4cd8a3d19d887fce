// The pipelined MFMA GEMM for gfx950: operand tiles stream from global memory straight into a ring of LDS stages,
// and eight waves in two groups take turns, one group's matrix-core work overlapping the other's LDS reads and load
// issue.
//
// A workgroup of 512 threads (eight waves, two on each SIMD) computes one BM x BN output tile (256 x 256 by
// default). Group 0 (waves 0-3) owns output rows 0 .. BM/2 - 1 of the tile and brings a's stages in; group 1 owns
// rows BM/2 .. BM - 1 and brings b's. Each wave holds a (BM/2) x (BN/4) block of accumulators. Every stage is 64
// bytes of k of every operand row (pipe.hpp), STAGES deep (4 x 32 KiB at 256 x 256), loaded by buffer_load ... lds
// so no register, transpose or LDS-write instruction of the wave is spent on it; M- or N-contiguous operands stay
// that way in LDS and are read with the LDS transpose reads.
//
// Iteration t has two phases, each ended by a workgroup barrier:
//   phase A: group 0 reads its fragments of stage t and issues the loads of stage t + STAGES - 1;
//            group 1 runs the MFMAs of stage t - 1 (fragments it read in the previous phase);
//   phase B: group 0 runs the MFMAs of stage t; group 1 reads its fragments of stage t and issues its loads.
// So on every SIMD one wave feeds the matrix core while the other waits on memory. Before the barrier that opens
// stage t + 1's first reads, each wave waits (vmcnt) for its own loads of that stage; a stage's buffer is refilled
// only after both groups' reads of it completed (lgkmcnt(0) before every barrier). No atomics: the result's bits do
// not depend on timing.
#include <hip/hip_runtime.h>
#include "kernels.hpp"
#include "mfma.hpp"
#include "pipe.hpp"
#include "ring.hpp"
#include "tile.hpp"

namespace cairn::gemm {
using namespace cairn::pipe;

template<class Sh, int OP, bool TA, bool TB>
__global__ void __launch_bounds__(512) pipe_gemm(Params p) {
  using M = Mfma<OP>;
  using Acc = typename M::Acc;
  constexpr bool AK = !TA, BKM = TB;
  constexpr int S = Sh::STAGES;
  __shared__ __attribute__((aligned(1024))) char lds[S * Sh::STAGE];

  const int t = threadIdx.x, lane = t & 63, gt = t & 255;
  const int wave = t >> 6, group = wave >> 2, w4 = wave & 3;
  int tm, tn;
  cairn::tile::tile_of(int(blockIdx.x), p.tiles_m, p.tiles_n, p.group, tm, tn);
  const int row0 = tm * Sh::BM, col0 = tn * Sh::BN;
  const cairn::tile::Panel pa = cairn::tile::panel(AK, row0, p.m, p.k, p.lda, Sh::ES);
  const cairn::tile::Panel pb = cairn::tile::panel(BKM, col0, p.n, p.k, p.ldb, Sh::ES);
  const char* a = static_cast<const char*>(p.a) + pa.start;
  const char* b = static_cast<const char*>(p.b) + pb.start;

  Dma dma;
  Loader<Sh, Sh::BM, AK, Dma> la;
  Loader<Sh, Sh::BN, BKM, Dma> lb;
  if(group == 0) la.setup(gt, row0, p.m, p.lda);
  else lb.setup(gt, col0, p.n, p.ldb);
  const int T = (p.k + Sh::BK - 1) / Sh::BK;
  auto issue = [&](int st) {
    char* stage = lds + (st % S) * Sh::STAGE;
    if(group == 0) la.issue(dma, a, pa.bytes, p.lda, st, p.k, stage, w4);
    else lb.issue(dma, b, pb.bytes, p.ldb, st, p.k, stage + Sh::A_BYTES, w4);
  };
  // Wait for this wave's loads of stage `next`, given the last stage it has issued: the loads of the stages after
  // `next` may stay in flight (the group's loads a stage: LOADS_A for group 0, LOADS_B for group 1).
  auto landed = [&](int next, int last) {
    const int ahead = last - next;
    if(group == 0) {
      if(ahead >= 2 && S >= 4) wait_loads<2 * Sh::LOADS_A>();
      else if(ahead >= 1) wait_loads<Sh::LOADS_A>();
      else wait_loads<0>();
    } else {
      if(ahead >= 2 && S >= 4) wait_loads<2 * Sh::LOADS_B>();
      else if(ahead >= 1) wait_loads<Sh::LOADS_B>();
      else wait_loads<0>();
    }
  };

  Acc acc[Sh::FM][Sh::FN];
#pragma unroll
  for(int i = 0; i < Sh::FM; ++i)
#pragma unroll
    for(int j = 0; j < Sh::FN; ++j) acc[i][j] = Acc{};
  u32x4 xa[2][Sh::FM], xb[2][Sh::FN];

  // A group's fragment reads of stage st. No wait follows them: the group's next phase is its MFMAs, which wait for
  // their own operands, and a stage's buffer is refilled only in a phase B after both groups' MFMAs of that stage.
  auto memory = [&](int st) {
    const char* stage = lds + (st % S) * Sh::STAGE;
#pragma unroll
    for(int s = 0; s < 2; ++s) {
      fragments<Sh, Sh::BM, AK, Sh::FM>(xa[s], stage, group * Sh::WTM, s, lane);
      fragments<Sh, Sh::BN, BKM, Sh::FN>(xb[s], stage + Sh::A_BYTES, w4 * Sh::WTN, s, lane);
    }
  };
  auto compute = [&]() {
#pragma unroll
    for(int s = 0; s < 2; ++s)
#pragma unroll
      for(int i = 0; i < Sh::FM; ++i)
#pragma unroll
        for(int j = 0; j < Sh::FN; ++j) acc[i][j] = M::step(xb[s][j], xa[s][i], acc[i][j]);
  };

  for(int st = 0; st < S - 1; ++st)
    if(st < T) issue(st);
  if(T > 0) landed(0, (S - 2 < T - 1 ? S - 2 : T - 1));
  barrier();
  for(int it = 0; it <= T; ++it) {
    if(group == 0) {
      if(it < T) memory(it);
    } else if(it > 0) {
      compute();
    }
    barrier();
    if(group == 0) {
      if(it < T) compute();
    } else if(it < T) {
      memory(it);
    }
    // Both groups refill stage it - 1's buffer with stage it + S - 1: group 0 computed stage it - 1 in the previous
    // phase B, group 1 in the phase A just ended.
    if(it < T && it + S - 1 < T) issue(it + S - 1);
    if(it + 1 < T) landed(it + 1, (it + S - 1 < T - 1 ? it + S - 1 : T - 1));
    barrier();
  }

  // Epilogue: block (i, j) of this wave, quad q of lane l: row m, columns n .. n+3.
#pragma unroll
  for(int i = 0; i < Sh::FM; ++i) {
    const int m = row0 + group * Sh::WTM + 32 * i + cairn::tile::acc_m(lane);
#pragma unroll
    for(int j = 0; j < Sh::FN; ++j)
#pragma unroll
      for(int q = 0; q < 4; ++q) {
        const int n = col0 + w4 * Sh::WTN + 32 * j + cairn::tile::acc_n(lane, q);
        if(m < p.m && n < p.n) store_quad(p, m, n, acc[i][j], q);
      }
  }
}

template<class Sh, int OP, bool TA, bool TB> hipError_t launch_pipe(const Params& p, hipStream_t s) {
  const unsigned grid = unsigned(p.tiles_m) * unsigned(p.tiles_n);
  hipLaunchKernelGGL((pipe_gemm<Sh, OP, TA, TB>), dim3(grid), dim3(512), 0, s, p);
  return hipGetLastError();
}

}  // namespace cairn::gemm

#define CAIRN_PIPE_INSTANCE(NAME, BM, BN, STAGES, OP, TA, TB)                                                     \
  hipError_t NAME(const cairn::gemm::Params& p, hipStream_t s) {                                                \
    return cairn::gemm::launch_pipe<cairn::pipe::Shape<BM, BN, (OP == cairn::gemm::OP_I8 ? 1 : 2), STAGES>, OP,  \
                                    TA, TB>(p, s);                                                                \
  }
#include "pipe_instances.inc"
