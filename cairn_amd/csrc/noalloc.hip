// cairn_gemm_run_static: cairn_gemm_run with the split last round's workspace taken from a scratch array the library
// holds on each GPU, for callers that cannot allocate (code under graph capture, tight serving loops, harnesses that
// forbid hipMalloc). Nothing here allocates, frees or makes a stream or event: the array is a file-scope device
// variable, present on every GPU the library runs on from its load to the process's end.
//
// Its device address is taken once per GPU, with that GPU current, by hipGetSymbolAddress; in host code the array's
// name is only a host-side stand-in, so that address, never the name, is what the kernels are given. Every call on
// one GPU uses the same array and leaves the last call's partial tiles in it: nothing in it needs to start at zero
// (a split writes every partial before its fixup reads it, in stream order), but two calls that may run at the same
// time on one GPU (on two streams, or from two threads) race on it.
#include <hip/hip_runtime.h>
#include <atomic>
#include <cstdint>
#include <mutex>
#include "../../include/cairn_gemm.h"

namespace {

static __device__ __align__(256) unsigned char scratch[CAIRN_GEMM_STATIC_SCRATCH];

constexpr int MAX_DEVICES = 64;
std::atomic<void*> where[MAX_DEVICES];  // the array's device address on each GPU, once taken
std::mutex taking;

// The scratch array's address on the current GPU, or null where the runtime refuses it.
void* scratch_here() {
  int device = 0;
  if(hipGetDevice(&device) != hipSuccess || device < 0 || device >= MAX_DEVICES) return nullptr;
  if(void* p = where[device].load(std::memory_order_acquire)) return p;
  const std::lock_guard<std::mutex> hold(taking);
  if(void* p = where[device].load(std::memory_order_relaxed)) return p;
  void* p = nullptr;
  if(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return nullptr;
  where[device].store(p, std::memory_order_release);
  return p;
}

}  // namespace

extern "C" __attribute__((visibility("default"))) int cairn_gemm_run_static(const cairn_gemm_desc* d, void* stream) {
  if(!d || d->version != CAIRN_GEMM_DESC_VERSION) return CAIRN_E_ARG;
  if(d->workspace) return CAIRN_E_ARG;  // the scratch is the library's: a caller's workspace has no place here
  void* at = scratch_here();
  if(!at) return CAIRN_E_HIP;
  cairn_gemm_desc mine = *d;
  mine.workspace = at;
  mine.workspace_bytes = CAIRN_GEMM_STATIC_SCRATCH;
  return cairn_gemm_run(&mine, stream);  // a split that needs more than the scratch answers CAIRN_E_SCRATCH
}
