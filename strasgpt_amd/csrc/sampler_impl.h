// The device sampler behind sampler_hip_t (include/sampler_hip.h): the
// reference sampler's parameters (include/sampler.h:19-31) and its state on
// the GPU: the xorshift64* state, the presence marks and the work buffers
// of sg::sample.
#pragma once

#include <hip/hip_runtime.h>

#include "kernels.h"

struct sampler_hip {
  int device = 0;
  int V = 0;
  float temperature = 0.0f;
  size_t top_k = 0;
  float top_p = 0.0f;
  float presence_penalty = 0.0f;
  unsigned long long seed = 0;
  hipStream_t stream = nullptr;  // for calls on host logits
  // device memory (one allocation per buffer)
  unsigned long long* rng = nullptr;
  unsigned char* presence = nullptr;
  unsigned char* keep = nullptr;
  float* y = nullptr;
  float* part = nullptr;
  unsigned *keys = nullptr, *keys_sorted = nullptr;
  int *vals = nullptr, *vals_sorted = nullptr;
  void* sort_temp = nullptr;
  size_t sort_temp_bytes = 0;
  float* scal = nullptr;
  int* nkeep = nullptr;
  float* argmax_v = nullptr;
  int* argmax_i = nullptr;
  float* x = nullptr;  // staging for host logits
  int* out = nullptr;
};

// sg::sample parameters for s over `logits` (device), the token written to
// out (and appended to seq, pos_inc bumped, when given).
sg::SampleParams sampler_params(sampler_hip* s, const float* logits, const int* prev, int prev_value,
                                int* out, int* seq, int* seq_len, int* pos_inc);
