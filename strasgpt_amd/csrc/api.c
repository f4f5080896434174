/*
 * Public StrasGPT C API (include/transformer.h, include/transformer_hip.h).
 *
 * The reference driver calls transformer_predict from every thread of an
 * OpenMP team and relies on orphaned worksharing ending in an implicit
 * barrier (reference source/strasgpt.c:209-232,
 * source/transformer.c:1724-1725). Here the device work runs inside one
 * orphaned `omp single`, whose implicit barrier makes every thread return
 * only after the logits are in the caller's buffer. Outside a parallel
 * region the call runs directly. This file is compiled with the host C
 * compiler's -fopenmp (GNU OpenMP ABI, which LLVM's libomp also provides),
 * keeping OpenMP out of the HIP code.
 */
#include <omp.h>
#include <stdlib.h>

#include "common.h"
#include "runtime.h"

transformer_t* transformer_from_safetensors(struct safetensors* safetensors) {
  return sg_from_safetensors(safetensors);
}

void transformer_free(transformer_t* transformer) { sg_free(transformer); }

void transformer_print(FILE* f, const transformer_t* transformer) {
  sg_print(f, transformer);
}

float* transformer_logits_malloc(transformer_t* transformer, size_t logits_count,
                                 size_t* vocabulary_len) {
  if (!transformer || !vocabulary_len) return NULL;
  *vocabulary_len = transformer->config->vocabulary_len;
  float* logits = malloc(logits_count * (*vocabulary_len) * sizeof(float));
  if (!logits) ST_DIE("failed to malloc for logits");
  return logits;
}

void transformer_predict(transformer_t* transformer, size_t token_count, int* token,
                         size_t logits_count, float* logits) {
  if (!transformer || !logits || token_count == 0 || logits_count == 0) return;
  if (omp_in_parallel()) {
    #pragma omp single
    sg_predict(transformer, token_count, token, logits_count, logits);
  } else {
    sg_predict(transformer, token_count, token, logits_count, logits);
  }
}

int transformer_predict_argmax(transformer_t* transformer, size_t token_count,
                               const int* token) {
  if (!transformer || token_count == 0) return -1;
  int result = -1;
  if (omp_in_parallel()) {
    /* result is shared through copyprivate */
    #pragma omp single copyprivate(result)
    result = sg_predict_argmax(transformer, token_count, token);
  } else {
    result = sg_predict_argmax(transformer, token_count, token);
  }
  return result;
}

size_t transformer_generate_greedy(transformer_t* transformer, size_t token_count,
                                   const int* token, size_t step_count, int eos_token_id,
                                   int* out, transformer_timing_t* timing) {
  if (!transformer || !out || token_count == 0 || step_count == 0) return 0;
  return sg_generate_greedy(transformer, token_count, token, step_count, eos_token_id,
                            out, timing);
}

size_t transformer_generate_sampled(transformer_t* transformer, size_t token_count,
                                    const int* token, size_t step_count, int eos_token_id,
                                    struct sampler_hip* sampler, int* out,
                                    transformer_timing_t* timing) {
  if (!transformer || !out || token_count == 0 || step_count == 0) return 0;
  return sg_generate_sampled(transformer, token_count, token, step_count, eos_token_id, sampler,
                             out, timing);
}

void transformer_reset(transformer_t* transformer) {
  if (transformer) sg_reset(transformer);
}

void transformer_capture_hidden(transformer_t* transformer, float* out, float* out_final) {
  if (transformer) sg_capture_hidden(transformer, out, out_final);
}

int transformer_set_prefill_precision(transformer_t* transformer, int mode) {
  return transformer ? sg_set_prefill_precision(transformer, mode) : -1;
}

const char* transformer_hip_version(void) { return sg_version(); }

int transformer_set_decode_mode(transformer_t* transformer, int mode) {
  return transformer ? sg_set_decode_mode(transformer, mode) : -1;
}

int transformer_set_kv_cache_format(transformer_t* transformer, int format) {
  return transformer ? sg_set_kv_cache_format(transformer, format) : -1;
}

void transformer_profile(transformer_t* transformer, int enable) {
  if (transformer) sg_profile(transformer, enable);
}

int transformer_profile_read(transformer_t* transformer, int kernel_class,
                             transformer_kernel_stat_t* out) {
  if (!transformer || !out) return -1;
  return sg_profile_read(transformer, kernel_class, out);
}

int transformer_kernel_rate(transformer_t* transformer, int kernel_class, int reps, double* avg_us,
                            double* bytes_per_launch) {
  if (!transformer || !avg_us || !bytes_per_launch) return -1;
  return sg_kernel_rate(transformer, kernel_class, reps, avg_us, bytes_per_launch);
}
