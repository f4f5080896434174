// Device token selection entry points (include/sampler_hip.h).
#include <limits.h>

#include <mutex>

#include <time.h>

#include "hip_check.h"
#include "kernels.h"
#include "sampler_hip.h"
#include "sampler_impl.h"

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

// ------------------------------------------------------ device sampler --
sg::SampleParams sampler_params(sampler_hip* s, const float* logits, const int* prev, int prev_value,
                                int* out, int* seq, int* seq_len, int* pos_inc) {
  sg::SampleParams p{};
  p.logits = logits;
  p.V = s->V;
  p.temperature = s->temperature;
  p.top_k = s->top_k > (size_t)s->V ? s->V : (int)s->top_k;
  p.top_p = s->top_p;
  p.penalty = s->presence_penalty;
  p.presence = s->presence;
  p.prev = prev;
  p.prev_value = prev_value;
  p.rng = s->rng;
  p.y = s->y;
  p.part = s->part;
  p.keys = s->keys;
  p.keys_sorted = s->keys_sorted;
  p.vals = s->vals;
  p.vals_sorted = s->vals_sorted;
  p.keep = s->keep;
  p.sort_temp = s->sort_temp;
  p.sort_temp_bytes = s->sort_temp_bytes;
  p.scal = s->scal;
  p.nkeep = s->nkeep;
  p.argmax_v = s->argmax_v;
  p.argmax_i = s->argmax_i;
  p.out = out;
  p.seq = seq;
  p.seq_len = seq_len;
  p.pos_inc = pos_inc;
  return p;
}

extern "C" sampler_hip_t* sampler_hip_build(size_t vocabulary_len, float temperature, size_t top_k,
                                            float top_p, unsigned long long seed) {
  if (vocabulary_len == 0 || vocabulary_len > (size_t)INT_MAX) ST_DIE("sampler: vocabulary_len out of range");
  if (!(temperature >= 0.0f)) ST_DIE("sampler: temperature must be >= 0");
  sampler_hip* s = new sampler_hip();
  HIP_CHECK(hipGetDevice(&s->device));
  const size_t V = vocabulary_len;
  s->V = (int)V;
  s->temperature = temperature;
  s->top_k = top_k;
  s->top_p = top_p;
  s->seed = seed ? seed : (unsigned long long)time(NULL);  // source/sampler.c:31-35
  HIP_CHECK(hipStreamCreate(&s->stream));
  HIP_CHECK(hipMalloc(&s->rng, sizeof(unsigned long long)));
  HIP_CHECK(hipMalloc(&s->presence, V));
  HIP_CHECK(hipMalloc(&s->keep, V));
  HIP_CHECK(hipMalloc(&s->y, V * sizeof(float)));
  HIP_CHECK(hipMalloc(&s->part, 512 * sizeof(float)));
  HIP_CHECK(hipMalloc(&s->keys, V * sizeof(unsigned)));
  HIP_CHECK(hipMalloc(&s->keys_sorted, V * sizeof(unsigned)));
  HIP_CHECK(hipMalloc(&s->vals, V * sizeof(int)));
  HIP_CHECK(hipMalloc(&s->vals_sorted, V * sizeof(int)));
  s->sort_temp_bytes = sg::sample_sort_temp_bytes(s->V);
  HIP_CHECK(hipMalloc(&s->sort_temp, s->sort_temp_bytes ? s->sort_temp_bytes : 1));
  HIP_CHECK(hipMalloc(&s->scal, 4 * sizeof(float)));
  HIP_CHECK(hipMalloc(&s->nkeep, sizeof(int)));
  HIP_CHECK(hipMalloc(&s->argmax_v, sg::argmax_blocks() * sizeof(float)));
  HIP_CHECK(hipMalloc(&s->argmax_i, sg::argmax_blocks() * sizeof(int)));
  HIP_CHECK(hipMalloc(&s->x, V * sizeof(float)));
  HIP_CHECK(hipMalloc(&s->out, sizeof(int)));
  HIP_CHECK(hipMemcpy(s->rng, &s->seed, sizeof(s->seed), hipMemcpyHostToDevice));
  HIP_CHECK(hipMemset(s->presence, 0, V));
  return s;
}

extern "C" void sampler_hip_free(sampler_hip_t* s) {
  if (!s) return;
  HIP_CHECK(hipStreamSynchronize(s->stream));
  void* bufs[] = {s->rng, s->presence, s->keep, s->y, s->part, s->keys, s->keys_sorted, s->vals,
                  s->vals_sorted, s->sort_temp, s->scal, s->nkeep, s->argmax_v, s->argmax_i, s->x, s->out};
  for (void* b : bufs)
    if (b) HIP_CHECK(hipFree(b));
  HIP_CHECK(hipStreamDestroy(s->stream));
  delete s;
}

extern "C" void sampler_hip_set_presence_penalty(sampler_hip_t* s, float penalty) {
  if (!s) ST_DIE("sampler: NULL sampler");
  s->presence_penalty = penalty;
}

extern "C" size_t sampler_hip_sample(sampler_hip_t* s, const float* logits, int token) {
  if (!s || !logits) ST_DIE("sampler: NULL sampler or logits");
  HIP_CHECK(hipSetDevice(s->device));
  HIP_CHECK(hipMemcpyAsync(s->x, logits, (size_t)s->V * sizeof(float), hipMemcpyHostToDevice, s->stream));
  sg::sample(sampler_params(s, s->x, nullptr, token, s->out, nullptr, nullptr, nullptr), s->stream);
  int tok = 0;
  HIP_CHECK(hipMemcpyAsync(&tok, s->out, sizeof(int), hipMemcpyDeviceToHost, s->stream));
  HIP_CHECK(hipStreamSynchronize(s->stream));
  return (size_t)tok;
}

extern "C" unsigned long long sampler_hip_rng_state(sampler_hip_t* s) {
  if (!s) ST_DIE("sampler: NULL sampler");
  unsigned long long v = 0;
  HIP_CHECK(hipSetDevice(s->device));
  HIP_CHECK(hipStreamSynchronize(s->stream));
  HIP_CHECK(hipMemcpy(&v, s->rng, sizeof(v), hipMemcpyDeviceToHost));
  return v;
}
