// Host check of mq::Div32 (the multiply-and-shift division of the kernels'
// index math) against integer division: every divisor 1..4096, 2^k and
// 2^k +- 1, sampled divisors up to 2^30, and indices at the edges (0, d - 1,
// d, multiples of d and their neighbours, 2^31 - 1) plus random ones below 2^31.
#include <cstdint>
#include <cstdio>
#include <random>
#include <vector>

#include "mq_launch.hpp"

int main() {
  std::vector<uint32_t> ds;
  for (uint32_t d = 1; d <= 4096; ++d) ds.push_back(d);
  for (int k = 12; k <= 30; ++k) {
    ds.push_back(1u << k);
    ds.push_back((1u << k) - 1);
    ds.push_back((1u << k) + 1);
  }
  std::mt19937_64 rng(12345);
  for (int n = 0; n < 2000; ++n) ds.push_back(1 + (uint32_t)(rng() % (1u << 30)));
  long bad = 0, checked = 0;
  for (uint32_t d : ds) {
    const mq::Div32 dv = mq::Div32::make(d);
    std::vector<uint32_t> is = {0u, 1u, d - 1, d, d + 1, 0x7FFFFFFFu, 0x7FFFFFFFu - d};
    const uint32_t top = 0x7FFFFFFFu / d;
    for (uint32_t m : {top, top - 1, top / 2 + 1}) {
      const uint64_t v = (uint64_t)m * d;
      if (v <= 0x7FFFFFFFu) { is.push_back((uint32_t)v); is.push_back((uint32_t)v - 1); }
      if (v + 1 <= 0x7FFFFFFFu) is.push_back((uint32_t)v + 1);
    }
    for (int n = 0; n < 200; ++n) is.push_back((uint32_t)(rng() & 0x7FFFFFFFu));
    for (uint32_t i : is) {
      if (i > 0x7FFFFFFFu) continue;
      ++checked;
      if (dv.div(i) != i / d) {
        if (bad < 5) std::printf("mismatch d=%u i=%u got %u want %u\n", d, i, dv.div(i), i / d);
        ++bad;
      }
    }
  }
  std::printf("checked %ld bad %ld\n", checked, bad);
  return bad != 0;
}
