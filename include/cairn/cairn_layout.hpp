// The two guards CAIRN-emitted fragment code wraps around a tile (src/cairn/compiler/device/fragments.py:346-372
// emits them; src/cairn/runtime/cairn_layout.hpp:10-20 states them): a coordinate is checked against its extent, and
// a tile's array against the largest offset its layout places, before any element is read or written. A broken one
// traps, on the host and in a device lane alike. And the CuTe-style swizzle a layout may name.
#pragma once
#include <cstddef>
#include "cairn_runtime.hpp"

namespace cr::layout {

CR_HD inline std::size_t within(std::size_t x, std::size_t extent) noexcept {
  if(x >= extent) trap();
  return x;
}

template<class T> CR_HD inline T* holding(T* data, std::size_t count, std::size_t cosize) noexcept {
  if(count < cosize) trap();
  return data;
}

// Swizzle<B, M, S>: the B bits from M + S up are XORed into the B bits from M up. With S >= 1 the bits that decide
// a flip never flip themselves, so the map is a permutation of offsets.
template<unsigned B, unsigned M, unsigned S> CR_HD constexpr std::size_t swizzle(std::size_t o) noexcept {
  return o ^ ((o >> S) & (((std::size_t(1) << B) - 1) << M));
}

}  // namespace cr::layout
