/*
 * Internal C interface between the OpenMP-aware public API (api.c, built
 * with the host C compiler) and the HIP runtime (runtime.hip). None of
 * these functions touch OpenMP: api.c runs them on one thread of the
 * caller's team.
 */
#ifndef STRASGPT_RUNTIME_H
#define STRASGPT_RUNTIME_H

#include <stddef.h>

#include "transformer.h"
#include "transformer_hip.h"

#ifdef __cplusplus
extern "C" {
#endif

transformer_t* sg_from_safetensors(struct safetensors* s);
void sg_free(transformer_t* t);
void sg_print(FILE* f, const transformer_t* t);
void sg_predict(transformer_t* t, size_t token_count, const int* token,
                size_t logits_count, float* logits);
int sg_predict_argmax(transformer_t* t, size_t token_count, const int* token);
size_t sg_generate_greedy(transformer_t* t, size_t token_count, const int* token,
                          size_t step_count, int eos, int* out,
                          transformer_timing_t* timing);
size_t sg_generate_sampled(transformer_t* t, size_t token_count, const int* token,
                           size_t step_count, int eos, struct sampler_hip* sampler, int* out,
                           transformer_timing_t* timing);
void sg_reset(transformer_t* t);
void sg_capture_hidden(transformer_t* t, float* out, float* out_final);
int sg_set_prefill_precision(transformer_t* t, int mode);
const char* sg_version(void);
int sg_set_decode_mode(transformer_t* t, int mode);
int sg_set_kv_cache_format(transformer_t* t, int format);
void sg_profile(transformer_t* t, int enable);
int sg_profile_read(transformer_t* t, int kernel_class, transformer_kernel_stat_t* out);
int sg_kernel_rate(transformer_t* t, int kernel_class, int reps, double* avg_us, double* bytes);

#ifdef __cplusplus
}
#endif

#endif
