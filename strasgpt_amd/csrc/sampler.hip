// Device token selection entry points (include/sampler_hip.h).
#include <limits.h>

#include "hip_check.h"
#include "kernels.h"
#include "sampler_hip.h"

extern "C" size_t sampler_argmax(const float* probability, size_t n) {
  if (!probability) ST_DIE("sampler_argmax: NULL probability");
  if (n == 0 || n > (size_t)INT_MAX) ST_DIE("sampler_argmax: n must be in [1, INT_MAX]");
  const int parts = sg::argmax_blocks();
  float *x = nullptr, *part_v = nullptr;
  int *part_i = nullptr, *out = nullptr;
  HIP_CHECK(hipMalloc(&x, n * sizeof(float)));
  HIP_CHECK(hipMalloc(&part_v, parts * sizeof(float)));
  HIP_CHECK(hipMalloc(&part_i, parts * sizeof(int)));
  HIP_CHECK(hipMalloc(&out, sizeof(int)));
  HIP_CHECK(hipMemcpy(x, probability, n * sizeof(float), hipMemcpyHostToDevice));
  sg::ArgmaxParams p{};
  p.x = x;
  p.n = (int)n;
  p.part_v = part_v;
  p.part_i = part_i;
  p.out = out;
  sg::argmax(p, nullptr);
  int best = 0;
  HIP_CHECK(hipMemcpy(&best, out, sizeof(int), hipMemcpyDeviceToHost));
  HIP_CHECK(hipFree(x));
  HIP_CHECK(hipFree(part_v));
  HIP_CHECK(hipFree(part_i));
  HIP_CHECK(hipFree(out));
  return (size_t)best;
}
