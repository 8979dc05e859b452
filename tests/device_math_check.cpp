// Host check of the branch-free approx_exp_fast against its loop form, over every float input
// in a stride of the 32-bit patterns (stride 1 = all 2^32).  Prints the mismatch count.
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "qwen_device_math.hpp"

int main(int argc, char** argv) {
  const unsigned long long stride = argc > 1 ? strtoull(argv[1], nullptr, 10) : 1;
  unsigned long long checked = 0, bad = 0;
  for (unsigned long long u = 0; u < (1ull << 32); u += stride) {
    const float v = qwen::bits_f32((uint32_t)u);
    const float a = qwen::approx_exp_fast(v), b = qwen::approx_exp_fast_ladder(v);
    ++checked;
    if (qwen::f32_bits(a) != qwen::f32_bits(b) && !(a != a && b != b)) {
      if (bad < 5) std::printf("mismatch at %08llx: %a vs %a\n", u, a, b);
      ++bad;
    }
  }
  std::printf("checked %llu mismatches %llu\n", checked, bad);
  return bad != 0;
}
