// The HIP execution layer (include/cairn/cairn_ops.hpp and cairn_hip_kernels.hpp over cairn_context.hpp) on the
// device, in programs shaped as CAIRN-emitted device code is: regions on the thread's context, reductions, scans and a compaction from
// its arena, the vector and staged plans, owners of device, pinned and unified storage, held runs, an enqueued call
// on the caller's stream, queued work on lent lanes, and a context with a budget of its own. Built by
// __graft_entry__.build() into tests/cpp/libexec_device.so; tests/test_gpu_exec.py calls it and checks every result
// against numpy. Every entry returns 0, or the number of the check that failed inside it.
#include <hip/hip_runtime.h>
#include <cstdint>
#include "cairn_gpu.hpp"

using namespace cr::gpu;

namespace {
// The fold the reductions and scans use: a sum in 64-bit integers, exact in any association order.
struct Add {
  __host__ __device__ long long operator()(long long a, long long b) const { return a + b; }
};
}  // namespace

// Regions on here(): a fresh buffer reads zeros; a fill; its sum; inclusive and exclusive scans with their totals;
// the positive elements' indices compacted; a vector plan (4 floats a lane) and a staged 3-point stencil.
extern "C" int exec_regions(std::size_t n, long long* sums, long long* inc, long long* exc, long long* kept,
                            std::size_t* used, float* vec, float* stencil) {
  Context& ctx = here();
  Buffer<int> x(n);
  int* p = x.data();
  sums[0] = reduce_on(ctx, n, 0LL, Add{}, [=] __host__ __device__(std::size_t i) { return (long long)p[i]; });
  run(ctx, n, [=] __device__(std::size_t i) { p[i] = int(i % 97) - 48; });
  sums[1] = reduce_on(ctx, n, 0LL, Add{}, [=] __host__ __device__(std::size_t i) { return (long long)p[i]; });
  Buffer<long long> si(n), se(n), k(n);
  sums[2] = scan_on<false>(ctx, si.data(), n, 0LL, Add{}, [=] __host__ __device__(std::size_t i) { return (long long)p[i]; });
  sums[3] = scan_on<true>(ctx, se.data(), n, 0LL, Add{}, [=] __host__ __device__(std::size_t i) { return (long long)p[i]; });
  copy_on(ctx, inc, si.data(), n, Dir::d2h);
  copy_on(ctx, exc, se.data(), n, Dir::d2h);
  *used = compact_on(ctx, k.data(), n, [=] __device__(std::size_t i) { return p[i] > 0; },
                     [=] __device__(std::size_t i) { return (long long)i; });
  copy_on(ctx, kept, k.data(), n, Dir::d2h);

  Buffer<float> v(n), s(n);
  float* pv = v.data();
  float* ps = s.data();
  run_vector<4>(
      ctx, n, aligned<4>(pv), [=] __device__(std::size_t i) { pv[i] = 0.5f * float(i); },
      [=] __device__(std::size_t i) {
        Chunk<float, 4> c;
        for(unsigned e = 0; e < 4; ++e) c[e] = 0.5f * float(i + e);
        c.store(pv + i);
      });
  copy_on(ctx, vec, pv, n, Dir::d2h);
  // out[i] = v[i - 1] + v[i] + v[i + 1], zeros outside: each block's tile of width + 2 floats in LDS.
  run_staged<1>(
      ctx, n,
      [=] __device__(std::size_t base, std::size_t w, std::size_t t, std::size_t b, unsigned char* tile) {
        float* f = reinterpret_cast<float*>(tile);
        for(std::size_t j = t; j < w; j += b) {
          const std::size_t at = base + j;  // element at - 1
          f[j] = at >= 1 && at - 1 < n ? pv[at - 1] : 0.0f;
        }
      },
      [=] __device__(std::size_t i, std::size_t base, std::size_t, unsigned char* tile) {
        const float* f = reinterpret_cast<const float*>(tile);
        const std::size_t j = i - base;
        ps[i] = (f[j] + f[j + 1]) + f[j + 2];
      },
      [](std::size_t width) { return tile_bytes<float>(width); });
  copy_on(ctx, stencil, ps, n, Dir::d2h);
  return 0;
}

// A held run of three regions, then an enqueued call on the caller's stream: out[0 .. n) = 2 (i + 1) after the
// held run; out[n .. 2n) = 7 i written by the enqueued call, which returns without waiting (the caller's stream is
// synchronized here before the copy back, as a C host would).
extern "C" int exec_streams(std::size_t n, void* stream, int* out, int* waited) {
  Context& ctx = here();
  Buffer<int> a(n), b(n);
  int* pa = a.data();
  int* pb = b.data();
  {
    Held held;
    run(ctx, n, [=] __device__(std::size_t i) { pa[i] = int(i); });
    run(ctx, n, [=] __device__(std::size_t i) { pa[i] += 1; });
    run(ctx, n, [=] __device__(std::size_t i) { pa[i] *= 2; });
  }
  copy_on(ctx, out, pa, n, Dir::d2h);
  {
    Enqueued call(stream);
    run(ctx, n, [=] __device__(std::size_t i) { pb[i] = 7 * int(i); });
  }
  // The enqueued work was queued on the caller's stream; nothing waited for it.
  *waited = hipStreamQuery(static_cast<hipStream_t>(stream)) == hipSuccess ? 1 : 0;
  check(hipStreamSynchronize(static_cast<hipStream_t>(stream)));
  copy_on(ctx, out + n, pb, n, Dir::d2h);
  return 0;
}

// Queued work on lent lanes: the second region follows the first's ticket; a copy follows the second.
extern "C" int exec_queue(std::size_t n, int* out) {
  Context& ctx = here();
  Buffer<int> a(n), b(n), c(n);
  int* pa = a.data();
  int* pb = b.data();
  Lent first = queue(ctx, n, [=] __device__(std::size_t i) { pa[i] = int(i) - 5; });
  Lent second = queue(ctx, n, [=] __device__(std::size_t i) { pb[i] = 3 * pa[i]; }, first);
  Lent third = queue_copy(ctx, c.data(), pb, n, Dir::d2d, second);
  wait(std::move(third));
  wait(std::move(second));
  wait(std::move(first));
  copy_on(ctx, out, c.data(), n, Dir::d2h);
  return ctx.tickets() == 0 ? 0 : 1;
}

// A context with a budget of its own: stream-ordered growth to a limit, over_budget past it, ok again within it.
// answers: a small reduce, a scan of `big` elements (whose held prefix alone passes the limit), another reduce;
// caps: the capacity after each; *total the last reduce's result.
extern "C" int exec_budget(std::size_t limit, std::size_t big, int* answers, std::size_t* caps, long long* total) {
  Context own(Budget{0, limit}, Allocation::stream_ordered);
  long long r = -1;
  answers[0] = int(reduce(own, r, 1000, 0LL, Add{}, [] __host__ __device__(std::size_t i) { return (long long)i; }));
  caps[0] = own.capacity();
  if(r != 499500) return 1;
  Buffer<long long> out(big);
  long long t = -1;
  answers[1] = int(cr::reuse::scan<false>(own, t, out.data(), big, 0LL, Add{},
                                          [] __host__ __device__(std::size_t i) { return (long long)i; }));
  caps[1] = own.capacity();
  if(answers[1] == int(Scratch::over_budget) && t != -1) return 2;  // over budget leaves the total alone
  answers[2] = int(reduce(own, r, 10, 0LL, Add{}, [] __host__ __device__(std::size_t i) { return (long long)i; }));
  caps[2] = own.capacity();
  *total = r;
  return own.tickets() == 0 ? 0 : 3;
}

// Owners of pinned and unified storage, and zero() at an odd address: out[0 .. 16) the unified squares the device
// wrote, read on the host (all -1 where the device reports no coherent access to managed memory: the unified owner
// is then not exercised); bytes: the 37 bytes after zeroing bytes 1 .. 35 of a buffer filled with 0xff.
extern "C" int exec_owners(int* out, unsigned char* bytes) {
  Context& ctx = here();
  Pinned<int> pin(16);
  for(int i = 0; i < 16; ++i)
    if(pin.data()[i] != 0) return 1;  // pinned storage starts zeroed
  int device = 0, managed = 0, coherent = 0;
  check(hipGetDevice(&device));
  check(hipDeviceGetAttribute(&managed, hipDeviceAttributeManagedMemory, device));
  check(hipDeviceGetAttribute(&coherent, hipDeviceAttributeConcurrentManagedAccess, device));
  if(managed && coherent) {
    Unified<int> uni(16);
    int* u = uni.data();
    run(ctx, 16, [=] __device__(std::size_t i) { u[i] = int(i * i); });
    for(int i = 0; i < 16; ++i) out[i] = u[i];
  } else {
    for(int i = 0; i < 16; ++i) out[i] = -1;
  }
  Buffer<unsigned char> z(37);
  unsigned char* pz = z.data();
  run(ctx, 37, [=] __device__(std::size_t i) { pz[i] = 0xff; });
  cr::reuse::synchronous(ctx, [&](hipStream_t s) { ctx.machine().zero(pz + 1, 35, s); });
  copy_on(ctx, bytes, pz, 37, Dir::d2h);
  return 0;
}

// The device-resident forms: reduce_to after a ticket (its total read after the ticket's wait), reduce_into and
// scan_into inside a held run (nothing waits until the run ends), a vector plan given a pointer off its chunk's
// width (the scalar lanes run instead), and a region of no indices. out: [reduce_to, reduce_into, exclusive scan
// of 0 .. 9 (10 values), vector plan over n floats from an odd float offset (n values)].
extern "C" int exec_resident(std::size_t n, long long* out, float* vec) {
  Context& ctx = here();
  Buffer<long long> cells(2), prefix(10);
  Buffer<float> v(n + 1);
  long long* pc = cells.data();
  Lent fill = queue(ctx, 2, [=] __device__(std::size_t i) { pc[i] = -1; });
  Scratch answer = Scratch::over_budget;
  Lent total = reduce_to(ctx, pc, 1000, 0LL, Add{}, [] __host__ __device__(std::size_t i) { return (long long)i; },
                         &answer, fill);
  wait(std::move(total));
  wait(std::move(fill));
  if(answer != Scratch::ok) return 1;
  {
    Held held;
    reduce_into(ctx, pc + 1, 100, 0LL, Add{}, [] __host__ __device__(std::size_t i) { return (long long)(2 * i); });
    scan_into<true>(ctx, prefix.data(), 10, 0LL, Add{}, [] __host__ __device__(std::size_t i) { return (long long)i; });
  }
  copy_on(ctx, out, pc, 2, Dir::d2h);
  copy_on(ctx, out + 2, prefix.data(), 10, Dir::d2h);
  float* odd = v.data() + 1;  // 4 bytes past a 256-byte boundary: not on a 16-byte chunk
  run_vector<4>(
      ctx, n, aligned<4>(odd), [=] __device__(std::size_t i) { odd[i] = 3.0f * float(i); },
      [=] __device__(std::size_t i) {
        Chunk<float, 4> c;
        for(unsigned e = 0; e < 4; ++e) c[e] = -1.0f;  // never taken for this pointer
        c.store(odd + i);
      });
  run(ctx, 0, [=] __device__(std::size_t i) { odd[i] = -7.0f; });  // no indices: nothing runs
  copy_on(ctx, vec, odd, n, Dir::d2h);
  return aligned<4>(odd) ? 2 : 0;
}
