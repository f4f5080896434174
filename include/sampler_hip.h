/*
 * Token selection on the device. The reference samples on the host
 * (source/sampler.c); these entry points run its selection rules on the
 * GPU.
 */
#ifndef SAMPLER_HIP_H
#define SAMPLER_HIP_H

#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

/* The reference's sample_argmax (source/sampler.c:92-102) on the device:
 * the first index holding the maximum of probability[0 .. n). A NaN never
 * wins over an earlier value, and a NaN at index 0 is never replaced (the
 * scan compares with a strict ">"). probability is a host array; each call
 * allocates device memory for a copy of it and for the per-block partial
 * results, runs two kernels on the GPU and frees the memory. Dies (like
 * every error of this library) when n is 0 or above INT_MAX. */
size_t sampler_argmax(const float* probability, size_t n);

/* sampler_argmax without any device allocation. No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). The values and the partial results are staged in one
 * statically allocated device array of about 1 MiB, which each GPU the
 * library runs on holds until the process ends. n is at most
 * SAMPLER_ARGMAX_NOALLOC_MAX (larger n dies with an error message). Every
 * call on one GPU uses that GPU's array: calls that overlap on the same
 * GPU (from several host threads) race and must be serialised by the
 * caller. Same result as sampler_argmax. */
#define SAMPLER_ARGMAX_NOALLOC_MAX 262144
size_t sampler_argmax_noalloc(const float* probability, size_t n);

/* The reference's sampler (include/sampler.h:19-38, source/sampler.c:14-337)
 * with its state on the GPU: temperature (0: greedy argmax), top_k (0: off),
 * top_p (outside (0, 1]: off), the xorshift64* generator seeded with seed
 * (0: time(NULL), like the reference's seed <= 0), the presence marks and a
 * presence penalty (0 unless set; the reference never sets it). One coin is
 * drawn per non-greedy call, as in the reference; draws follow its steps
 * with its per-element arithmetic and differ only in summation order
 * (softmax, top-p and multinomial running sums), i.e. only when the coin or
 * top_p lies within that rounding of a boundary. Equal probabilities rank
 * by index. The sampler lives on the device that is current when it is
 * built. */
typedef struct sampler_hip sampler_hip_t;
sampler_hip_t* sampler_hip_build(size_t vocabulary_len, float temperature, size_t top_k,
                                 float top_p, unsigned long long seed);
void sampler_hip_free(sampler_hip_t* sampler);
void sampler_hip_set_presence_penalty(sampler_hip_t* sampler, float penalty);
/* The reference's sampler_sample(sampler, logits, token) on a host array of
 * vocabulary_len logits (not modified) and the previous token (marked
 * present; < 0: none). Returns the drawn token. */
size_t sampler_hip_sample(sampler_hip_t* sampler, const float* logits, int token);
/* The generator state (after the draws so far). */
unsigned long long sampler_hip_rng_state(sampler_hip_t* sampler);

#ifdef __cplusplus
}
#endif

#endif /* SAMPLER_HIP_H */
