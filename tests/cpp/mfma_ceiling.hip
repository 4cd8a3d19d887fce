// An MFMA-only ceiling for the tiled GEMM kernels: how fast the matrix cores of every CU run when a workgroup does
// nothing but issue MFMAs on operands held in registers, with no memory traffic in its loop. The operands are
// patterns the caller uploads (random data of the GEMM's type), so the instructions draw the power they draw in a
// GEMM on such data. Each workgroup is four waves, one a SIMD, and holds 96 KiB of LDS so that only one fits a CU: a
// grid of one workgroup per CU keeps every SIMD of the chip issuing. Each wave runs CHAINS independent accumulators,
// so no MFMA waits for the result of the one before it.
//
// Wave 0 of each workgroup stamps the shader clock counter (s_memtime) and the constant-rate wall clock
// (s_memrealtime) around its loop: cycles over wall time is that CU's clock while it ran, and cycles over the MFMAs
// a wave issued is the cycles an MFMA took. Built by __graft_entry__.build() into tests/cpp/libmfma_ceiling.so;
// `python bench.py --only ceiling` runs it.
#include <hip/hip_runtime.h>
#include <cstdint>

namespace {

typedef std::uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));

constexpr int CHAINS = 4;
constexpr int THREADS = 256;
constexpr int HOLD = 96 * 1024;

enum Type { BF16 = 0, I8 = 1, F8E4M3 = 2 };

template<int T> struct Op;
template<> struct Op<BF16> {  // v_mfma_f32_32x32x16_bf16
  using Acc = f32x16;
  __device__ static Acc step(u32x4 x, u32x4 y, Acc c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, x), __builtin_bit_cast(bf16x8, y), c,
                                                   0, 0, 0);
  }
};
template<> struct Op<I8> {  // v_mfma_i32_32x32x32_i8
  using Acc = i32x16;
  __device__ static Acc step(u32x4 x, u32x4 y, Acc c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(__builtin_bit_cast(i32x4, x), __builtin_bit_cast(i32x4, y), c, 0, 0,
                                                 0);
  }
};
template<> struct Op<F8E4M3> {  // v_mfma_f32_32x32x64_f8f6f4, E4M3 both sides: 32 bytes of k an operand
  using Acc = f32x16;
  __device__ static Acc step(u32x4 x, u32x4 y, Acc c) {
    const i32x8 a = {int(x[0]), int(x[1]), int(x[2]), int(x[3]), int(y[0]), int(y[1]), int(y[2]), int(y[3])};
    const i32x8 b = {int(y[0]), int(y[1]), int(y[2]), int(y[3]), int(x[0]), int(x[1]), int(x[2]), int(x[3])};
    return __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c, 0, 0, 0, 0, 0, 0);
  }
};

// ops: `count` 16-byte patterns; out: one float a thread (the sum of its accumulators, so nothing is dropped);
// stamps: four counters a workgroup (cycles before, cycles after, wall before, wall after).
template<int T>
__global__ void __launch_bounds__(THREADS) ceiling(const u32x4* ops, int count, int iterations, float* out,
                                                   unsigned long long* stamps) {
  __shared__ unsigned char hold[HOLD];
  const int t = blockIdx.x * THREADS + threadIdx.x;
  u32x4 x[CHAINS], y[CHAINS];
#pragma unroll
  for(int c = 0; c < CHAINS; ++c) {
    x[c] = ops[unsigned(t * 2 * CHAINS + 2 * c) % unsigned(count)];
    y[c] = ops[unsigned(t * 2 * CHAINS + 2 * c + 1) % unsigned(count)];
  }
  hold[threadIdx.x] = static_cast<unsigned char>(t);
  typename Op<T>::Acc acc[CHAINS] = {};
  __syncthreads();
  const unsigned long long c0 = __builtin_amdgcn_s_memtime(), w0 = __builtin_amdgcn_s_memrealtime();
  for(int i = 0; i < iterations; ++i) {
#pragma unroll
    for(int c = 0; c < CHAINS; ++c) acc[c] = Op<T>::step(x[c], y[c], acc[c]);
  }
  const unsigned long long c1 = __builtin_amdgcn_s_memtime(), w1 = __builtin_amdgcn_s_memrealtime();
  float s = float(hold[(threadIdx.x + 1) % THREADS]);
#pragma unroll
  for(int c = 0; c < CHAINS; ++c)
#pragma unroll
    for(int e = 0; e < 16; ++e) s += float(acc[c][e]);
  out[t] = s;
  if(threadIdx.x == 0) {
    stamps[4 * blockIdx.x + 0] = c0;
    stamps[4 * blockIdx.x + 1] = c1;
    stamps[4 * blockIdx.x + 2] = w0;
    stamps[4 * blockIdx.x + 3] = w1;
  }
}

}  // namespace

// Queue the probe: `workgroups` workgroups of 256 threads, `iterations` rounds of CHAINS MFMAs a wave. out holds
// workgroups * 256 floats, stamps workgroups * 4 counters, ops `count` 16-byte patterns. Returns a hipError_t.
extern "C" __attribute__((visibility("default"))) int ceiling_launch(int type, int workgroups, int iterations,
                                                                     const void* ops, int count, void* out,
                                                                     void* stamps, void* stream) {
  if(type < BF16 || type > F8E4M3 || workgroups <= 0 || iterations <= 0 || count <= 0 || !ops || !out || !stamps)
    return int(hipErrorInvalidValue);
  const auto s = static_cast<hipStream_t>(stream);
  const auto* o = static_cast<const u32x4*>(ops);
  auto* f = static_cast<float*>(out);
  auto* st = static_cast<unsigned long long*>(stamps);
  if(type == BF16) hipLaunchKernelGGL(ceiling<BF16>, dim3(workgroups), dim3(THREADS), 0, s, o, count, iterations, f, st);
  else if(type == I8) hipLaunchKernelGGL(ceiling<I8>, dim3(workgroups), dim3(THREADS), 0, s, o, count, iterations, f, st);
  else hipLaunchKernelGGL(ceiling<F8E4M3>, dim3(workgroups), dim3(THREADS), 0, s, o, count, iterations, f, st);
  return int(hipGetLastError());
}

// The MFMAs a wave issues in one launch, and the multiply-adds (x2 for FLOP) each one does.
extern "C" __attribute__((visibility("default"))) int ceiling_chains() { return CHAINS; }
extern "C" __attribute__((visibility("default"))) long ceiling_flop_per_mfma(int type) {
  return type == BF16 ? 2L * 32 * 32 * 16 : type == I8 ? 2L * 32 * 32 * 32 : 2L * 32 * 32 * 64;
}

// The wall clock's rate in kHz (s_memrealtime), or 0 where the runtime does not say.
extern "C" __attribute__((visibility("default"))) int ceiling_wall_khz() {
  int device = 0, khz = 0;
  if(hipGetDevice(&device) != hipSuccess) return 0;
  if(hipDeviceGetAttribute(&khz, hipDeviceAttributeWallClockRate, device) != hipSuccess) return 0;
  return khz;
}
