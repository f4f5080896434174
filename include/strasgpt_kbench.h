/*
 * Measurement and test hooks of libstrasgpt_hip (no reference
 * counterpart: the reference has no GPU kernels). Each call allocates its
 * own device buffers. Returns 0, or -1 for invalid arguments.
 */
#ifndef STRASGPT_KBENCH_H
#define STRASGPT_KBENCH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* The device MXFP4 decode used by the expert kernels, on `nblocks` host
 * blocks of 32 values (16 code bytes, element 2i in the low nibble of byte
 * i, and one E8M0 scale byte each): out[32 b + i] = value i of block b. */
int strasgpt_kbench_mxfp4_decode(const uint8_t* codes, const uint8_t* scales, int nblocks,
                                 float* out);

/* The same blocks through the grouped prefill GEMM's conversion (MXFP4 to
 * packed bf16 pairs, as it fills the matrix-core tiles), widened back to
 * fp32: equal to the fp32 decode wherever the value fits bf16 (all of them:
 * two significant bits). */
int strasgpt_kbench_mxfp4_decode_bf16(const uint8_t* codes, const uint8_t* scales, int nblocks,
                                      float* out);

/* Copy of `bytes` (multiple of 16) between two device buffers: one warm-up
 * launch of copy_probe_kernel (reads and writes exactly `bytes`), then
 * `iters` launches back to back between two events; *avg_us is the average
 * per launch. The calibration kernel for HBM traffic counters. */
int strasgpt_kbench_copy(size_t bytes, int iters, double* avg_us);

/* Sustained bf16 matrix-core rate: every wave of waves_per_simd (1 or 2) per
 * SIMD on every CU issues 16 x iters v_mfma_f32_32x32x16_bf16 over 8
 * independent accumulators, operands cycled over 8 register fragments of
 * random finite bf16 values (random_operands) or one constant pattern; one
 * warm-up launch, then `launches` launches between two events; *tflops is
 * the achieved rate. The reference point for the prefill GEMMs: the rate
 * and, read with the clock counters, the clock the chip holds when operands
 * toggle like real data. */
int strasgpt_kbench_mfma(int random_operands, int waves_per_simd, int iters, int launches,
                         double* tflops);

/* The device sampler's sort on n host pairs (key, index): a stable
 * descending sort by key (equal keys in index order), the order the top-k
 * and top-p cuts walk. keys_out[r] = the r-th key, index_out[r] its index.
 * 1 <= n <= 1 << 26. */
int strasgpt_kbench_sort_desc(const uint32_t* keys, int n, uint32_t* keys_out, int32_t* index_out);

#ifdef __cplusplus
}
#endif

#endif
