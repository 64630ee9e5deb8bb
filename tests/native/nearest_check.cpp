// nearest_check.cpp — the windowed FP4 / NF4 table search (common.hpp
// nearest_window) against nearest16, the reference's full search, on every
// f32 bit pattern (test infrastructure; built host-only and run by
// tests/test_nearest_window.py).  Prints the mismatches it finds (at most
// 20) and "nearest_check: ok <count>" when there are none.
#include <atomic>
#include <cstdio>
#include <cstring>
#include <thread>
#include <vector>

#include "common.hpp"

namespace {

std::atomic<long> g_bad{0};

template <bool NF4>
void sweep(uint64_t lo, uint64_t hi) {
  constexpr wh::TabSearch t = wh::make_tab_search<NF4>();
  long bad = 0;
  for (uint64_t u = lo; u < hi; ++u) {
    float r;
    const uint32_t b = (uint32_t)u;
    std::memcpy(&r, &b, 4);
    const uint32_t want = wh::nearest16(t.val, r), got = wh::nearest_window<NF4>(t, r);
    if (want != got) {
      if (g_bad.fetch_add(1) < 20)
        std::printf("%s r=%a (0x%08x): nearest16 %u, window %u\n", NF4 ? "nf4" : "fp4", (double)r, b, want, got);
      ++bad;
    }
  }
}

}  // namespace

int main(int argc, char **argv) {
  const int threads = argc > 1 ? std::atoi(argv[1]) : 8;
  const uint64_t total = 1ull << 32, step = total / (uint64_t)threads;
  for (int nf4 = 0; nf4 < 2; ++nf4) {
    std::vector<std::thread> pool;
    for (int i = 0; i < threads; ++i) {
      const uint64_t lo = (uint64_t)i * step, hi = i + 1 == threads ? total : lo + step;
      pool.emplace_back(nf4 ? sweep<true> : sweep<false>, lo, hi);
    }
    for (auto &th : pool) th.join();
  }
  if (g_bad.load() != 0) {
    std::printf("nearest_check: %ld mismatches\n", g_bad.load());
    return 1;
  }
  std::printf("nearest_check: ok %llu\n", 2ull * total);
  return 0;
}
