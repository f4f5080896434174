// Measurement and test hooks (include/strasgpt_kbench.h): the calibration
// copy for HBM traffic counters, the sustained matrix-core rate probe, and
// the expert kernels' MXFP4 decode on host-supplied blocks.
#include "device_common.h"
#include "hip_check.h"
#include "kernels.h"
#include "strasgpt_kbench.h"

namespace {

// Deterministic non-zero fill of n floats.
__global__ void fill_f32(float* x, size_t n) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    x[i] = (float)(i % 1021) * 0.001f + 1.0f;
}

// Plain copy dst = src of n float4 (the calibration kernel for HBM traffic
// counters: it reads and writes exactly 16 n bytes).
__global__ __launch_bounds__(256) void copy_probe_kernel(const float4* __restrict__ src,
                                                         float4* __restrict__ dst, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    dst[i] = src[i];
}

}  // namespace

extern "C" int strasgpt_kbench_sort_desc(const uint32_t* keys, int n, uint32_t* keys_out, int32_t* index_out) {
  if (!keys || !keys_out || !index_out || n < 1 || n > sg::kSortMax) return -1;
  unsigned *k, *ko;
  int* vo;
  void* tmp;
  const size_t tb = sg::sample_sort_temp_bytes(n);
  HIP_CHECK(hipMalloc(&k, (size_t)n * 4));
  HIP_CHECK(hipMalloc(&ko, (size_t)n * 4));
  HIP_CHECK(hipMalloc(&vo, (size_t)n * 4));
  HIP_CHECK(hipMalloc(&tmp, tb));
  HIP_CHECK(hipMemcpy(k, keys, (size_t)n * 4, hipMemcpyHostToDevice));
  sg::sort_pairs_desc(k, nullptr, n, ko, vo, tmp, nullptr);
  HIP_CHECK(hipMemcpy(keys_out, ko, (size_t)n * 4, hipMemcpyDeviceToHost));
  HIP_CHECK(hipMemcpy(index_out, vo, (size_t)n * 4, hipMemcpyDeviceToHost));
  HIP_CHECK(hipFree(k));
  HIP_CHECK(hipFree(ko));
  HIP_CHECK(hipFree(vo));
  HIP_CHECK(hipFree(tmp));
  return 0;
}

extern "C" int strasgpt_kbench_copy(size_t bytes, int iters, double* avg_us) {
  if (bytes < 16 || bytes % 16 || iters <= 0 || !avg_us) return -1;
  hipStream_t s;
  HIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  float4 *a, *b;
  HIP_CHECK(hipMalloc(&a, bytes));
  HIP_CHECK(hipMalloc(&b, bytes));
  hipLaunchKernelGGL(fill_f32, dim3(1024), dim3(256), 0, s, (float*)a, bytes / 4);
  const size_t n = bytes / 16;
  hipEvent_t e0, e1;
  HIP_CHECK(hipEventCreate(&e0));
  HIP_CHECK(hipEventCreate(&e1));
  hipLaunchKernelGGL(copy_probe_kernel, dim3(2048), dim3(256), 0, s, a, b, n);  // warm-up
  HIP_CHECK(hipEventRecord(e0, s));
  for (int i = 0; i < iters; i++)
    hipLaunchKernelGGL(copy_probe_kernel, dim3(2048), dim3(256), 0, s, a, b, n);
  HIP_CHECK(hipEventRecord(e1, s));
  HIP_CHECK(hipGetLastError());
  HIP_CHECK(hipEventSynchronize(e1));
  float ms = 0.f;
  HIP_CHECK(hipEventElapsedTime(&ms, e0, e1));
  *avg_us = ms * 1e3 / iters;
  HIP_CHECK(hipEventDestroy(e0));
  HIP_CHECK(hipEventDestroy(e1));
  HIP_CHECK(hipFree(a));
  HIP_CHECK(hipFree(b));
  HIP_CHECK(hipStreamDestroy(s));
  return 0;
}

// Sustained v_mfma_f32_32x32x16_bf16 issue: 8 accumulator chains per wave,
// operands cycled over 8 A and 8 B fragments per lane (random finite bf16
// bits, or one constant pattern), no memory traffic until the final store.
// The attainable matrix-core rate (and, read with the clock counters, the
// clock the chip holds) when operands toggle as real data does.
namespace {
__device__ unsigned probe_hash(unsigned x) {
  x ^= x >> 16;
  x *= 0x7feb352dU;
  x ^= x >> 15;
  x *= 0x846ca68bU;
  x ^= x >> 16;
  return x;
}
typedef unsigned probe_u32x4 __attribute__((ext_vector_type(4)));
__global__ __launch_bounds__(256) void mfma_probe_kernel(float* out, int iters, int random) {
  bf16x8 a[8], b[8];
#pragma unroll
  for (int j = 0; j < 8; j++) {
    probe_u32x4 ua, ub;
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const unsigned r = random ? probe_hash(threadIdx.x * 977u + j * 131u + i * 7u + blockIdx.x) : 0x3f803f80u;
      const unsigned q = random ? probe_hash(r + 12345u) : 0x3f803f80u;
      ua[i] = (r & 0x807f807fu) | 0x3f003f00u;  // magnitudes in [0.5, 1): no overflow
      ub[i] = (q & 0x807f807fu) | 0x3f003f00u;
    }
    a[j] = __builtin_bit_cast(bf16x8, ua);
    b[j] = __builtin_bit_cast(bf16x8, ub);
  }
  f32x16 c[8];
#pragma unroll
  for (int j = 0; j < 8; j++)
#pragma unroll
    for (int e = 0; e < 16; e++) c[j][e] = 0.0f;
  for (int it = 0; it < iters; it++) {
#pragma unroll
    for (int j = 0; j < 8; j++) c[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[j], b[(j + 3) & 7], c[j], 0, 0, 0);
#pragma unroll
    for (int j = 0; j < 8; j++) c[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a[(j + 5) & 7], b[j], c[j], 0, 0, 0);
  }
  float sum = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; j++) sum += c[j][0];
  out[blockIdx.x * 256 + threadIdx.x] = sum;
}
}  // namespace

extern "C" int strasgpt_kbench_mfma(int random_operands, int waves_per_simd, int iters, int launches,
                                    double* tflops) {
  if (waves_per_simd < 1 || waves_per_simd > 2 || iters <= 0 || launches <= 0 || !tflops) return -1;
  int cus = 0;
  HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0));
  const int blocks = cus * waves_per_simd;  // 4 waves per block: one per SIMD
  hipStream_t s;
  HIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  float* out;
  HIP_CHECK(hipMalloc(&out, (size_t)blocks * 256 * sizeof(float)));
  hipEvent_t e0, e1;
  HIP_CHECK(hipEventCreate(&e0));
  HIP_CHECK(hipEventCreate(&e1));
  hipLaunchKernelGGL(mfma_probe_kernel, dim3(blocks), dim3(256), 0, s, out, iters, random_operands);  // warm-up
  HIP_CHECK(hipEventRecord(e0, s));
  for (int i = 0; i < launches; i++)
    hipLaunchKernelGGL(mfma_probe_kernel, dim3(blocks), dim3(256), 0, s, out, iters, random_operands);
  HIP_CHECK(hipEventRecord(e1, s));
  HIP_CHECK(hipGetLastError());
  HIP_CHECK(hipEventSynchronize(e1));
  float ms = 0.f;
  HIP_CHECK(hipEventElapsedTime(&ms, e0, e1));
  *tflops = (double)launches * blocks * 4 * iters * 16 * 32768.0 / (ms * 1e-3) / 1e12;
  HIP_CHECK(hipEventDestroy(e0));
  HIP_CHECK(hipEventDestroy(e1));
  HIP_CHECK(hipFree(out));
  HIP_CHECK(hipStreamDestroy(s));
  return 0;
}

static int mxfp4_decode_hook(const uint8_t* codes, const uint8_t* scales, int nblocks, float* out,
                             int bf16_tiles) {
  if (nblocks <= 0 || !codes || !scales || !out) return -1;
  uint8_t *dc, *ds;
  float* dout;
  HIP_CHECK(hipMalloc(&dc, (size_t)nblocks * 16));
  HIP_CHECK(hipMalloc(&ds, (size_t)nblocks));
  HIP_CHECK(hipMalloc(&dout, (size_t)nblocks * 32 * sizeof(float)));
  HIP_CHECK(hipMemcpy(dc, codes, (size_t)nblocks * 16, hipMemcpyHostToDevice));
  HIP_CHECK(hipMemcpy(ds, scales, (size_t)nblocks, hipMemcpyHostToDevice));
  sg::mxfp4_decode(dc, ds, nblocks, dout, bf16_tiles, 0);
  HIP_CHECK(hipMemcpy(out, dout, (size_t)nblocks * 32 * sizeof(float), hipMemcpyDeviceToHost));
  HIP_CHECK(hipFree(dc));
  HIP_CHECK(hipFree(ds));
  HIP_CHECK(hipFree(dout));
  return 0;
}

extern "C" int strasgpt_kbench_mxfp4_decode(const uint8_t* codes, const uint8_t* scales, int nblocks,
                                            float* out) {
  return mxfp4_decode_hook(codes, scales, nblocks, out, 0);
}

extern "C" int strasgpt_kbench_mxfp4_decode_bf16(const uint8_t* codes, const uint8_t* scales, int nblocks,
                                                 float* out) {
  return mxfp4_decode_hook(codes, scales, nblocks, out, 1);
}
