// The conventions the multiply's C++ surface keeps from CAIRN's runtime (src/cairn/runtime/cairn_runtime.hpp:59-114,
// 194-205): a failed guard aborts the process (no exceptions, no return codes), extents multiply with an overflow
// check, a view is a pointer and an element count, and a read-write view may not overlap another view of a call.
#pragma once
#include <cstddef>
#include <cstdint>
#include <cstdio>
#include <cstdlib>

// Host-and-device functions: CR_HD marks what both compile (the spelling of src/cairn/runtime/cairn_runtime.hpp:18-24).
#if defined(__HIPCC__)
#define CR_HD __host__ __device__
#else
#define CR_HD
#endif

namespace cr {

// A broken guard stops the program: the host aborts; a device lane raises the wave's trap, which ends the kernel
// with an error the next wait on its stream reports (src/cairn/runtime/cairn_runtime.hpp:59-70 does the same with
// CUDA's trap).
[[noreturn]] CR_HD inline void trap() noexcept {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_trap();
#else
  std::abort();
#endif
}

// a * b, or a trap where it overflows.
template<class T> inline T mul(T a, T b) noexcept {
  T r;
  if(__builtin_mul_overflow(a, b, &r)) trap();
  return r;
}

// A view handed in through C: `count` elements at `data`. A null pointer holds nothing, and a pointer off its
// element's alignment is refused.
template<class T> inline void view(const T* data, std::size_t count) noexcept {
  if(count && !data) trap();
  if(reinterpret_cast<std::uintptr_t>(data) % alignof(T)) trap();
  if(count > static_cast<std::size_t>(PTRDIFF_MAX) / sizeof(T)) trap();
}

// A read-write view and another view of the same call share no byte.
template<class T, class U> inline void disjoint(const T* w, std::size_t wn, const U* r, std::size_t rn) noexcept {
  if(!wn || !rn) return;
  const auto w0 = reinterpret_cast<std::uintptr_t>(w), r0 = reinterpret_cast<std::uintptr_t>(r);
  const auto w1 = w0 + wn * sizeof(T), r1 = r0 + rn * sizeof(U);
  if(w0 < r1 && r0 < w1) trap();
}

}  // namespace cr
