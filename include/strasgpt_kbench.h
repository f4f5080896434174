/*
 * Kernel micro-benchmarks of libstrasgpt_hip (no reference counterpart:
 * the reference has no GPU kernels). Each call allocates its own device
 * buffers, fills them with seeded values, times `iters` launches of one
 * launch-shape variant with HIP events on one stream (average per-launch
 * duration in microseconds), and checks the result against a naive
 * one-thread-per-output kernel (largest |error| / largest |reference|).
 * Returns 0, or -1 for an invalid variant or shape.
 */
#ifndef STRASGPT_KBENCH_H
#define STRASGPT_KBENCH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Decode GEMV y = W x, W bf16 [N][K] (dual: SwiGLU of two matrices). */
int strasgpt_kbench_gemv(int n, int k, int dual, int variant, int iters,
                         double* avg_us, double* rel_err);
int strasgpt_kbench_gemv_variants(void);
/* Same with options in `flags`. Launches cycle through enough weight
 * copies (over 1 GiB) that every launch streams its weights from HBM
 * rather than from the Infinity Cache.
 *   bit 0: input RMSNorm prologue;
 *   bit 1: before each timed launch, an untimed kernel reads one word per
 *          64 KiB of that launch's weights (warms address translation);
 *   bit 2: time all launches back to back between two events instead of
 *          one event pair per launch;
 *   bit 3: one weight copy re-read by every launch (Infinity Cache hits
 *          when it fits). */
int strasgpt_kbench_gemv2(int n, int k, int dual, int flags, int variant, int iters,
                          double* avg_us, double* rel_err);

/* Prefill GEMM C = A W^T, A fp32 [M][K], W bf16 [N][K]; precision 0 is
 * bf16x2 (split activations), 1 is bf16; adding 2 evicts the caches before
 * each timed launch (operands come from HBM, as in a prefill pass). */
int strasgpt_kbench_gemm(int m, int n, int k, int precision, int variant, int iters,
                         double* avg_us, double* rel_err);
int strasgpt_kbench_gemm_variants(void);

/* The device MXFP4 decode used by the expert kernels, on `nblocks` host
 * blocks of 32 values (16 code bytes, element 2i in the low nibble of byte
 * i, and one E8M0 scale byte each): out[32 b + i] = value i of block b. */
int strasgpt_kbench_mxfp4_decode(const uint8_t* codes, const uint8_t* scales, int nblocks,
                                 float* out);

/* Copy of `bytes` (multiple of 16) between two device buffers, `iters`
 * launches of copy_probe_kernel (reads and writes exactly `bytes` each):
 * the calibration kernel for HBM traffic counters. */
int strasgpt_kbench_copy(size_t bytes, int iters, double* avg_us);

/* Grid barrier cost: one cooperative launch of `blocks` x 256 threads doing
 * `rounds` barriers, each block writing `words` values before each barrier.
 * fence 0: plain stores, no fences, no check; 1: fenced barrier, plain
 * stores and loads; 2: fence-free barrier, agent-coherent stores and loads.
 * Modes 1 and 2 count stale values read after each barrier in *bad_reads.
 * Returns -2 if the blocks cannot all be resident. */
int strasgpt_kbench_barrier(int blocks, int rounds, int fence, int words,
                            double* us_per_round, int* bad_reads, int* timed_out);

/* Causal prefill attention over T queries after P cached positions
 * (synthetic fp32 queries and cache); variant 0 is the split-bf16
 * matrix-core kernel, 1 the fp32 matrix-core kernel. */
int strasgpt_kbench_attn_prefill(int T, int P, int q_heads, int kv_heads, int hd, int variant,
                                 int iters, double* avg_us);

#ifdef __cplusplus
}
#endif

#endif
