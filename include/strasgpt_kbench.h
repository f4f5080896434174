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

#ifdef __cplusplus
extern "C" {
#endif

/* Decode GEMV y = W x, W bf16 [N][K] (dual: SwiGLU of two matrices). */
int strasgpt_kbench_gemv(int n, int k, int dual, int variant, int iters,
                         double* avg_us, double* rel_err);
int strasgpt_kbench_gemv_variants(void);
/* Same with the input RMSNorm prologue (norm != 0). Launches cycle
 * through enough weight copies (over 1 GiB) that every launch streams its
 * weights from HBM rather than from the Infinity Cache. */
int strasgpt_kbench_gemv2(int n, int k, int dual, int norm, int variant, int iters,
                          double* avg_us, double* rel_err);

/* Prefill GEMM C = A W^T, A fp32 [M][K], W bf16 [N][K]; precision 0 is
 * bf16x2 (split activations), 1 is bf16. */
int strasgpt_kbench_gemm(int m, int n, int k, int precision, int variant, int iters,
                         double* avg_us, double* rel_err);
int strasgpt_kbench_gemm_variants(void);

#ifdef __cplusplus
}
#endif

#endif
