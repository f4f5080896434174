// Device token selection entry points (include/sampler_hip.h).
#include <limits.h>

#include <mutex>

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

// ------------------------------------------------ no-allocation variant --
// sampler_argmax_noalloc stages the caller's values and the partial
// results in one statically allocated device array instead of hipMalloc'd
// buffers. Each GPU the library runs on holds its own copy of the array
// until the process ends; host code reaches a device's copy only through
// the address hipGetSymbolAddress returns for it (taken once per device,
// with that device current).
namespace {

constexpr size_t kNoallocMaxValues = (size_t)1 << 18;  // SAMPLER_ARGMAX_NOALLOC_MAX
constexpr size_t kNoallocParts = 1024;                 // >= sg::argmax_blocks()
constexpr size_t kScratchBytes = kNoallocMaxValues * sizeof(float) +
                                 kNoallocParts * (sizeof(float) + sizeof(int)) + 256;

__device__ __align__(256) unsigned char scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex scratch_mutex;
void* scratch_ptr[kMaxDevices] = {};

// The current device's copy of `scratch`.
void* device_scratch() {
  int dev = 0;
  HIP_CHECK(hipGetDevice(&dev));
  if (dev < 0 || dev >= kMaxDevices) ST_DIE("sampler_argmax_noalloc: device index out of range");
  std::lock_guard<std::mutex> lock(scratch_mutex);
  if (!scratch_ptr[dev]) {
    void* p = nullptr;
    HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    if (!p) ST_DIE("sampler_argmax_noalloc: no device address for the scratch array");
    scratch_ptr[dev] = p;
  }
  return scratch_ptr[dev];
}

}  // namespace

extern "C" size_t sampler_argmax_noalloc(const float* probability, size_t n) {
  static_assert(SAMPLER_ARGMAX_NOALLOC_MAX == kNoallocMaxValues, "header limit");
  if (!probability) ST_DIE("sampler_argmax_noalloc: NULL probability");
  if (n == 0) ST_DIE("sampler_argmax_noalloc: n must be at least 1");
  if (n > kNoallocMaxValues) ST_DIE("sampler_argmax_noalloc: n exceeds SAMPLER_ARGMAX_NOALLOC_MAX (262144)");
  const int parts = sg::argmax_blocks();
  if (parts <= 0 || (size_t)parts > kNoallocParts) ST_DIE("sampler_argmax_noalloc: too many partial results");
  // Layout in the scratch array: values [n], partial values [parts],
  // partial indices [parts], the result (all fully written before read).
  unsigned char* base = (unsigned char*)device_scratch();
  float* x = (float*)base;
  float* part_v = (float*)(base + kNoallocMaxValues * sizeof(float));
  int* part_i = (int*)(part_v + kNoallocParts);
  int* out = part_i + kNoallocParts;
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
  return (size_t)best;
}
