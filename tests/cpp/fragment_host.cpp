// The MFMA fragments' host model (include/cairn/cairn_fragment.hpp) as CAIRN's host build runs it: one wave of 64
// threads, each holding every fragment whole, loads A and B through their tiles' layouts (row-major, padded,
// swizzled, column-major), multiplies and accumulates over two k-steps, and stores the accumulator, each lane only
// the elements the device gives it. Checked, as tests/runtime/fragment_runtime.cpp checks the reference's families:
//
// - every output equals the reference loop's (its old value, then its products in increasing k, each sum an f32
//   rounding; int8: exact integers), bit for bit;
// - every element is written exactly once, and each lane holds M * N / 64 of them;
// - a lane's value v (get/set) is the element `element` names, and that element's holder is the lane.
//
// Built with -fsanitize=thread by the test, so two lanes writing one element would also be reported.
// "trap" as the first argument asks get for a value past the share instead: the process must abort.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <thread>
#include <vector>
#include "cairn_fragment.hpp"
#include "cairn_layout.hpp"

namespace {
using namespace cr::frag;

std::uint64_t mix(std::uint64_t x) {
  x ^= x >> 29;
  x *= 0xbf58476d1ce4e5b9ULL;
  x ^= x >> 32;
  return x;
}

// Operand values: multiples of 1/16 in [-2, 2] (exact in every format here, every sum exact in f32), or int8.
template<class T> T value(std::uint64_t seed) {
  if constexpr(std::is_same_v<T, std::int8_t>) return T(std::int64_t(mix(seed) % 255) - 127);
  else return cr::fp::narrow<T>(double(std::int64_t(mix(seed) % 65) - 32) / 16.0);
}

int failures = 0;

// One layout of an R x C tile: an offset for each element.
struct Tile {
  std::size_t rows, cols, pitch;
  bool by_columns;   // element (r, c) at c * pitch + r
  unsigned swizzle;  // 0: none; else Swizzle<swizzle, 3, 3> on the offset
  std::size_t operator()(std::size_t r, std::size_t c) const {
    const std::size_t o = by_columns ? c * pitch + r : r * pitch + c;
    return swizzle == 1 ? cr::layout::swizzle<1, 3, 3>(o) : swizzle == 2 ? cr::layout::swizzle<2, 3, 3>(o) : o;
  }
  std::size_t cosize() const {
    std::size_t most = 0;
    for(std::size_t r = 0; r < rows; ++r)
      for(std::size_t c = 0; c < cols; ++c) most = std::max(most, (*this)(r, c));
    return most + 1;
  }
};

// C += A * B over two k-steps of one M x N x K shape: A is M x 2K, B is 2K x N, through the given tiles.
template<class T, int M, int N, int K> void wave(const char* what, Tile ta, Tile tb, Tile tc) {
  using H = held_t<T>;
  std::vector<T> as(ta.cosize()), bs(tb.cosize());
  std::vector<H> cs(tc.cosize()), want(M * N);
  for(int r = 0; r < M; ++r)
    for(int p = 0; p < 2 * K; ++p) as[ta(r, p)] = value<T>(1 + r * 2 * K + p);
  for(int p = 0; p < 2 * K; ++p)
    for(int c = 0; c < N; ++c) bs[tb(p, c)] = value<T>(90001 + p * N + c);
  for(int r = 0; r < M; ++r)
    for(int c = 0; c < N; ++c) {
      H acc = H(std::int64_t(mix(77 + r * N + c) % 9) - 4) / H(std::is_integral_v<H> ? 1 : 4);
      cs[tc(r, c)] = acc;
      for(int p = 0; p < 2 * K; ++p) {
        const H x = widen(as[ta(r, p)]) * widen(bs[tb(p, c)]);
        acc = std::is_integral_v<H> ? H(std::int32_t(std::uint32_t(acc) + std::uint32_t(x))) : acc + x;
      }
      want[r * N + c] = acc;
    }
  // The lanes store here; an element no lane writes keeps the sentinel, one written twice is counted.
  const H sentinel = std::is_integral_v<H> ? H(0x5a5a5a5a) : H(NAN);
  std::vector<H> out(cs.size(), sentinel);
  std::vector<int> writes(cs.size(), 0);
  auto at = [](const Tile& t, std::size_t dr, std::size_t dc) {
    return [t, dr, dc](std::size_t r, std::size_t c) { return t(r + dr, c + dc); };
  };
  std::vector<std::thread> lanes;
  std::vector<int> share_errors(WAVE, 0);
  for(unsigned lane = 0; lane < WAVE; ++lane)
    lanes.emplace_back([&, lane] {
      auto c = loaded<MfmaFragment<Role::acc, H, M, N, K>>(cs.data(), at(tc, 0, 0), tc.pitch, !tc.by_columns, true);
      for(int s = 0; s < 2; ++s) {
        const auto a = loaded<MfmaFragment<Role::a, T, M, N, K>>(as.data(), at(ta, 0, s * K), ta.pitch, !ta.by_columns, true);
        const auto b = loaded<MfmaFragment<Role::b, T, M, N, K>>(bs.data(), at(tb, s * K, 0), tb.pitch, !tb.by_columns, true);
        c = multiplied(c, a, b);
      }
      // get and set name this lane's own elements.
      for(std::size_t v = 0; v < std::size_t(values<M, N>); ++v) {
        const std::size_t e = element<M, N>(lane, v);
        if(holder<M, N>(e / N, e % N) != lane) ++share_errors[lane];
        const H before = get(c, v, lane);
        if(!(before == c.e[e])) ++share_errors[lane];
        const auto d = set(c, v, before + H(1), lane);
        if(!(get(d, v, lane) == before + H(1))) ++share_errors[lane];
      }
      stored(c, out.data(), at(tc, 0, 0), tc.pitch, !tc.by_columns, lane);
    });
  for(auto& l : lanes) l.join();
  for(unsigned lane = 0; lane < WAVE; ++lane)
    if(share_errors[lane]) {
      std::printf("%s: lane %u's get/set do not name its own elements\n", what, lane);
      ++failures;
      return;
    }
  for(int r = 0; r < M; ++r)
    for(int c = 0; c < N; ++c) {
      const H got = out[tc(r, c)];
      if(!(got == want[r * N + c])) {
        std::printf("%s: element (%d, %d) is %.9g, the reference %.9g\n", what, r, c, double(got), double(want[r * N + c]));
        ++failures;
        return;
      }
    }
  for(unsigned lane = 0; lane < WAVE; ++lane) {  // each lane holds M * N / 64 elements, and each element one lane
    int held = 0;
    for(int r = 0; r < M; ++r)
      for(int c = 0; c < N; ++c) held += holder<M, N>(r, c) == lane;
    if(held != values<M, N>) {
      std::printf("%s: lane %u holds %d elements\n", what, lane, held);
      ++failures;
    }
  }
  std::printf("ok %s\n", what);
}
}  // namespace

int main(int argc, char** argv) {
  if(argc > 1 && std::strcmp(argv[1], "trap") == 0) {
    MfmaFragment<Role::acc, float, 16, 16, 32> f{};
    std::printf("%g\n", double(get(f, values<16, 16>, 0)));  // past the share: aborts
    return 0;
  }
  // 32 x 32 x 16: A is 32 x 32, B 32 x 32, C 32 x 32; 16 x 16 x 32: A 16 x 64, B 64 x 16; int8 32 x 32 x 32.
  wave<cr::bf16, 32, 32, 16>("bf16 32x32x16 row-major", {32, 32, 32, false, 0}, {32, 32, 32, false, 0},
                             {32, 32, 32, false, 0});
  wave<cr::f16, 32, 32, 16>("f16 32x32x16 padded, B by columns", {32, 32, 40, false, 0}, {32, 32, 40, true, 0},
                            {32, 32, 36, false, 0});
  wave<cr::bf16, 32, 32, 16>("bf16 32x32x16 swizzled A", {32, 32, 32, false, 1}, {32, 32, 32, false, 2},
                             {32, 32, 32, true, 0});
  wave<cr::bf16, 16, 16, 32>("bf16 16x16x32 row-major", {16, 64, 64, false, 0}, {64, 16, 16, false, 0},
                             {16, 16, 16, false, 0});
  wave<cr::f16, 16, 16, 32>("f16 16x16x32 padded", {16, 64, 72, false, 0}, {64, 16, 24, false, 0},
                            {16, 16, 20, false, 0});
  wave<std::int8_t, 32, 32, 32>("int8 32x32x32 row-major", {32, 64, 64, false, 0}, {64, 32, 32, false, 0},
                                {32, 32, 32, false, 0});
  wave<std::int8_t, 32, 32, 32>("int8 32x32x32 B by columns", {32, 64, 80, false, 0}, {64, 32, 64, true, 0},
                                {32, 32, 40, false, 0});
  if(failures) return 1;
  std::printf("every lane's fragments equal the reference\n");
  return 0;
}
