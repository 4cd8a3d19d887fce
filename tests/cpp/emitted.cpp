// A translation unit shaped like what CAIRN emits around a device mma_unordered (src/cairn/compiler/device/tensor.py
// :69-82, lower/codegen.py:486-512): the runtime headers by their bare names, the checked C entry (views, then the
// disjointness of the read-write view), then the lean body's call on the thread's execution context. Built with the
// host compiler against include/cairn and linked against libcairn_gemm_gfx950.so, it shows that emitted code needs
// nothing beyond this include set and this library. tests/test_cpp_surface.py compiles and links it; nothing runs.
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

int main() { return 0; }
