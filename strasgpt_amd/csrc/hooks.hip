// Measurement and test hooks (include/strasgpt_kbench.h): the calibration
// copy for HBM traffic counters and the expert kernels' MXFP4 decode on
// host-supplied blocks.
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

extern "C" int strasgpt_kbench_mxfp4_decode(const uint8_t* codes, const uint8_t* scales, int nblocks,
                                            float* out) {
  if (nblocks <= 0 || !codes || !scales || !out) return -1;
  uint8_t *dc, *ds;
  float* dout;
  HIP_CHECK(hipMalloc(&dc, (size_t)nblocks * 16));
  HIP_CHECK(hipMalloc(&ds, (size_t)nblocks));
  HIP_CHECK(hipMalloc(&dout, (size_t)nblocks * 32 * sizeof(float)));
  HIP_CHECK(hipMemcpy(dc, codes, (size_t)nblocks * 16, hipMemcpyHostToDevice));
  HIP_CHECK(hipMemcpy(ds, scales, (size_t)nblocks, hipMemcpyHostToDevice));
  sg::mxfp4_decode(dc, ds, nblocks, dout, 0);
  HIP_CHECK(hipMemcpy(out, dout, (size_t)nblocks * 32 * sizeof(float), hipMemcpyDeviceToHost));
  HIP_CHECK(hipFree(dc));
  HIP_CHECK(hipFree(ds));
  HIP_CHECK(hipFree(dout));
  return 0;
}
