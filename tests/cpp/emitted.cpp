// A translation unit shaped like what CAIRN emits around a device mma_unordered (src/cairn/compiler/device/tensor.py
// :69-82, lower/codegen.py:486-512): the runtime headers by their bare names, the checked C entry (views, then the
// disjointness of the read-write view), then the lean body's call on the thread's execution context.
// tests/test_cpp_surface.py builds it two ways with the host compiler:
//   - against include/cairn and libcairn_gemm_gfx950.so: emitted code needs nothing beyond this include set and this
//     library (linked, not run);
//   - with -DCAIRN_EMULATE (`cairn build --emulate`): no library and no GPU, the device work on the host. Then main()
//     runs the entries on host arrays for every storage float and checks them bit for bit against the host multiply,
//     and a held run, an enqueued call and a GEMM descriptor on the emulated machine.
#include "cairn_runtime.hpp"
#include "cairn_tensor.hpp"
#include "cairn_gpu.hpp"

static void mma_lean(std::size_t m, std::size_t n, std::size_t k, float* v_c, std::size_t n_c, const cr::bf16* v_a,
                     std::size_t n_a, const cr::bf16* v_b, std::size_t n_b) noexcept {
  cr::tensor::launch<cr::bf16>(cr::gpu::here(), m, n, k, v_c, n_c, v_a, n_a, v_b, n_b);
}

extern "C" void cf_emitted_mma(std::size_t m, std::size_t n, std::size_t k, std::size_t n_c, float* v_c,
                               std::size_t n_a, const cairn_bf16* a, std::size_t n_b, const cairn_bf16* b) {
  const cr::bf16* v_a = reinterpret_cast<const cr::bf16*>(a);
  const cr::bf16* v_b = reinterpret_cast<const cr::bf16*>(b);
  cr::view(v_c, n_c);
  cr::view(v_a, n_a);
  cr::view(v_b, n_b);
  cr::disjoint(v_c, n_c, v_a, n_a);
  cr::disjoint(v_c, n_c, v_b, n_b);
  mma_lean(m, n, k, v_c, n_c, v_a, n_a, v_b, n_b);
}

extern "C" void cq_emitted_mma(void* stream, std::size_t m, std::size_t n, std::size_t k, std::size_t n_c, float* v_c,
                               std::size_t n_a, const cairn_bf16* a, std::size_t n_b, const cairn_bf16* b) {
  cr::gpu::Enqueued on(stream);
  cf_emitted_mma(m, n, k, n_c, v_c, n_a, a, n_b, b);
}

#if defined(CAIRN_EMULATE)
#include <cstdio>
#include <cstring>
#include <vector>

namespace {
int failures = 0;
void expect(bool ok, const char* what) {
  std::printf("%s %s\n", ok ? "ok" : "FAIL", what);
  if(!ok) ++failures;
}
// ((e + seed) * mul % 61 - 30) / 16, the reference's device-test generator (tests/soundness/test_tensor.py:201-202).
double drawn(std::size_t e, std::size_t seed, unsigned long long mul) {
  return double(long((e + seed) * mul % 61) - 30) / 16.0;
}
template<class A> std::vector<A> matrix(std::size_t count, std::size_t seed, unsigned long long mul) {
  std::vector<A> v(count);
  for(std::size_t e = 0; e < count; ++e) v[e] = cr::fp::narrow<A>(drawn(e, seed, mul));
  return v;
}
template<class A> bool same_as_host(std::size_t m, std::size_t n, std::size_t k, std::size_t seed) {
  const auto a = matrix<A>(m * k, seed, 2654435761ull), b = matrix<A>(k * n, seed * 3, 40503ull);
  std::vector<float> got(m * n), want(m * n);
  for(std::size_t e = 0; e < m * n; ++e) got[e] = want[e] = float(drawn(e, 99 + seed, 7)) / 2;
  cr::tensor::launch<A>(cr::gpu::here(), m, n, k, got.data(), got.size(), a.data(), a.size(), b.data(), b.size());
  cr::tensor::multiply<A>(m, n, k, want.data(), want.size(), a.data(), a.size(), b.data(), b.size());
  return std::memcmp(got.data(), want.data(), got.size() * sizeof(float)) == 0;
}
template<class A> bool every_shape() {
  const std::size_t shapes[][4] = {{1, 1, 1, 1}, {65, 63, 33, 2}, {130, 70, 100, 3}, {64, 64, 32, 4}, {72, 80, 96, 5},
                                   {129, 136, 8, 6}, {3, 4, 0, 7}};
  bool ok = true;
  for(const auto& s : shapes) ok &= same_as_host<A>(s[0], s[1], s[2], s[3]);
  return ok;
}
}  // namespace

int main() {
  expect(every_shape<cr::f16>(), "f16: launch on the emulated machine is the host multiply, bit for bit");
  expect(every_shape<cr::bf16>(), "bf16: the same");
  expect(every_shape<cr::f8e4m3>(), "f8e4m3: the same");
  expect(every_shape<cr::f8e5m2>(), "f8e5m2: the same");
  {  // the C entries, held and enqueued, as a C host calls them
    const std::size_t m = 20, n = 12, k = 16;
    const auto a = matrix<cr::bf16>(m * k, 1, 2654435761ull), b = matrix<cr::bf16>(k * n, 3, 40503ull);
    std::vector<float> c(m * n, 0.0f), want(m * n, 0.0f);
    for(int i = 0; i < 2; ++i)
      cr::tensor::multiply<cr::bf16>(m, n, k, want.data(), want.size(), a.data(), a.size(), b.data(), b.size());
    const auto* ca = reinterpret_cast<const cairn_bf16*>(a.data());
    const auto* cb = reinterpret_cast<const cairn_bf16*>(b.data());
    {
      const cr::gpu::Held held;
      cf_emitted_mma(m, n, k, c.size(), c.data(), a.size(), ca, b.size(), cb);
    }
    cq_emitted_mma(nullptr, m, n, k, c.size(), c.data(), a.size(), ca, b.size(), cb);
    expect(c == want && !cr::gpu::here().enqueued() && cr::gpu::here().tickets() == 0,
           "the checked entry in a held run, then the enqueued entry, each add a b once");
  }
  {  // a descriptor: TN layout, bias, ReLU, bf16 out; and int8 to int32
    const std::size_t m = 8, n = 12, k = 10;
    const auto at = matrix<cr::bf16>(k * m, 5, 2654435761ull), b = matrix<cr::bf16>(k * n, 6, 40503ull);
    std::vector<float> bias(n);
    for(std::size_t j = 0; j < n; ++j) bias[j] = float(drawn(j, 8, 3));
    std::vector<cr::bf16> out(m * n);
    cairn_gemm_desc d{};
    d.version = CAIRN_GEMM_DESC_VERSION;
    d.ab_type = CAIRN_TYPE_BF16;
    d.c_type = CAIRN_TYPE_BF16;
    d.trans_a = 1;
    d.m = m, d.n = n, d.k = k;
    d.a = at.data(), d.b = b.data(), d.c = out.data();
    d.act = CAIRN_ACT_RELU;
    d.bias = bias.data();
    d.bias_type = CAIRN_TYPE_F32;
    cr::tensor::gemm(cr::gpu::here(), d);
    bool ok = true;
    for(std::size_t i = 0; i < m; ++i)
      for(std::size_t j = 0; j < n; ++j) {
        float v = 0.0f;
        for(std::size_t p = 0; p < k; ++p) v = v + float(at[p * m + i]) * float(b[p * n + j]);
        v = v + bias[j];
        v = v < 0.0f ? 0.0f : v;
        ok &= out[i * n + j].bits == cr::fp::narrow<cr::bf16>(double(v)).bits;
      }
    std::vector<signed char> ai(m * k), bi(k * n);
    for(std::size_t e = 0; e < ai.size(); ++e) ai[e] = (signed char)(long(e * 37 % 255) - 127);
    for(std::size_t e = 0; e < bi.size(); ++e) bi[e] = (signed char)(long(e * 91 % 255) - 127);
    std::vector<int> acc(m * n, -1);
    cairn_gemm_desc q{};
    q.version = CAIRN_GEMM_DESC_VERSION;
    q.ab_type = CAIRN_TYPE_I8;
    q.c_type = CAIRN_TYPE_I32;
    q.m = m, q.n = n, q.k = k;
    q.a = ai.data(), q.b = bi.data(), q.c = acc.data();
    cr::tensor::gemm(cr::gpu::here(), q);
    for(std::size_t i = 0; i < m; ++i)
      for(std::size_t j = 0; j < n; ++j) {
        long s = 0;
        for(std::size_t p = 0; p < k; ++p) s += long(ai[i * k + p]) * long(bi[p * n + j]);
        ok &= acc[i * n + j] == int(s);
      }
    expect(ok, "a descriptor's GEMM: the stated steps in order (TN, bias, ReLU, bf16), and int8 exact");
  }
  std::printf("%d failures\n", failures);
  return failures ? 1 : 0;
}
#else
int main() { return 0; }
#endif
