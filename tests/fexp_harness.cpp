// Host build of the softmax exponential (synaptik_amd/csrc/fexp.h) checked against the
// reference expression (float)exp((double)t) (CpuSoftmaxReferenceKernel.java:104-146).
// Prints: evaluated, differing, max_ulp, exact_outside_fast_range (1/0), nan_ok (1/0).
#define __host__
#define __device__
#include "../synaptik_amd/csrc/fexp.h"
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>

static int64_t ordinal(float f) {
  int32_t i;
  memcpy(&i, &f, 4);
  return i < 0 ? -(int64_t)(i & 0x7fffffff) : (int64_t)i;
}

int main(int argc, char** argv) {
  const uint64_t stride = argc > 1 ? strtoull(argv[1], nullptr, 10) : 257;
  int64_t n = 0, diff = 0, max_ulp = 0;
  int exact_outside = 1, nan_ok = 1;
  for (uint64_t u = 0; u < 0x100000000ull; u += stride) {
    const uint32_t bits = (uint32_t)u;
    float t;
    memcpy(&t, &bits, 4);
    const float got = shk::exp_f32(t), want = (float)exp((double)t);
    if (std::isnan(want) || std::isnan(got)) {
      if (std::isnan(want) != std::isnan(got)) nan_ok = 0;
      continue;
    }
    ++n;
    const int64_t d = llabs(ordinal(got) - ordinal(want));
    if (d) ++diff;
    if (d > max_ulp) max_ulp = d;
    if (!(t >= -87.0f && t <= 88.0f) && d) exact_outside = 0;
  }
  printf("%lld %lld %lld %d %d\n", (long long)n, (long long)diff, (long long)max_ulp, exact_outside,
         nan_ok);
  return 0;
}
