// Host build of the library's expf restatement (c0ven_amd/csrc/device_math.h), compared with libm's expf on every
// float (or on every stride-th one), and its sigmoid and SwiGLU step against the same formulas on libm's expf.
// Prints "mismatches N checked M". Built and run by tests/test_expf.py.
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "../c0ven_amd/csrc/device_math.h"

static const uint64_t kTab[32] = {C0VEN_EXP2_TAB_VALUES};

static float bits(uint32_t u) {
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}
static uint32_t ubits(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  return u;
}

int main(int argc, char **argv) {
  const uint64_t stride = argc > 1 ? std::strtoull(argv[1], nullptr, 10) : 1;
  unsigned long long bad = 0, checked = 0;
#pragma omp parallel for reduction(+ : bad, checked) schedule(static)
  for (long long i = 0; i < (1ll << 32); i += (long long)stride) {
    const float x = bits((uint32_t)i);
    const float a = c0ven::expf_libm(x, kTab), b = std::exp(x);
    const bool same = ubits(a) == ubits(b) || (std::isnan(a) && std::isnan(b));
    bad += !same;
    if (!same && bad < 4) std::fprintf(stderr, "x %a: %a vs libm %a\n", x, a, b);
    checked++;
    if ((i / (long long)stride) % 97 == 0) {
      const float s = c0ven::sigmoid_libm(x, kTab), sr = 1.0f / (1.0f + std::exp(-x));
      const float g = c0ven::swiglu_one(x, 0.75f, 0.0f, kTab), gr = x / (1.0f + std::exp(-x)) * 0.75f;
      bad += !(ubits(s) == ubits(sr) || (std::isnan(s) && std::isnan(sr)));
      bad += !(ubits(g) == ubits(gr) || (std::isnan(g) && std::isnan(gr)));
    }
  }
  std::printf("mismatches %llu checked %llu\n", bad, checked);
  return bad != 0;
}
