// Kernel micro-benchmarks (include/strasgpt_kbench.h): event-timed launch
// variants of the GEMV and GEMM kernels on seeded data, each checked
// against a naive reference kernel.
#include <math.h>

#include <vector>

#include "device_common.h"
#include "hip_check.h"
#include "kernels.h"
#include "strasgpt_kbench.h"

namespace sg {
int gemv_variant_count();
void gemv_variant(const GemvParams& p, bool dual, int v, hipStream_t s);
int gemm_variant_count();
void gemm_variant(const GemmParams& p, int precision, int v, hipStream_t s);
}  // namespace sg

namespace {

__device__ __forceinline__ uint32_t hash32(uint32_t x) {
  x ^= x >> 16;
  x *= 0x7feb352dU;
  x ^= x >> 15;
  x *= 0x846ca68bU;
  x ^= x >> 16;
  return x;
}

// bf16 values uniform in about [-0.03, 0.03); fp32 values in [-1, 1).
__global__ void fill_bf16(uint16_t* w, size_t n, uint32_t seed) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    const float v = ((hash32((uint32_t)i * 2654435761u + seed) >> 8) / 16777216.0f - 0.5f) * 0.06f;
    w[i] = f32_to_bf16_rne(v);
  }
}
__global__ void fill_f32(float* x, size_t n, uint32_t seed) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    x[i] = (hash32((uint32_t)i * 2246822519u + seed) >> 8) / 8388608.0f - 1.0f;
}

__global__ void naive_gemv(const uint16_t* w, const uint16_t* w2, const float* x, int n, int k,
                           float* y) {
  const int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= n) return;
  float a = 0.0f, b = 0.0f;
  for (int i = 0; i < k; i++) {
    a = fmaf(bf16_to_f32(w[(size_t)r * k + i]), x[i], a);
    if (w2) b = fmaf(bf16_to_f32(w2[(size_t)r * k + i]), x[i], b);
  }
  y[r] = w2 ? a * (1.0f / (1.0f + expf(-a))) * b : a;
}

__global__ void naive_gemm(const float* a, const uint16_t* w, int m, int n, int k, float* c) {
  const int col = blockIdx.x * blockDim.x + threadIdx.x, row = blockIdx.y;
  if (col >= n) return;
  float acc = 0.0f;
  for (int i = 0; i < k; i++) acc = fmaf(a[(size_t)row * k + i], bf16_to_f32(w[(size_t)col * k + i]), acc);
  c[(size_t)row * n + col] = acc;
}

double rel_error(const std::vector<float>& got, const std::vector<float>& ref) {
  double e = 0, m = 0;
  for (size_t i = 0; i < ref.size(); i++) {
    e = fmax(e, fabs((double)got[i] - ref[i]));
    m = fmax(m, fabs((double)ref[i]));
  }
  return m > 0 ? e / m : e;
}

template <typename F>
double time_launches(hipStream_t s, int iters, F launch) {
  launch();
  launch();
  std::vector<hipEvent_t> ev(2 * iters);
  for (auto& e : ev) HIP_CHECK(hipEventCreate(&e));
  for (int i = 0; i < iters; i++) {
    HIP_CHECK(hipEventRecord(ev[2 * i], s));
    launch();
    HIP_CHECK(hipEventRecord(ev[2 * i + 1], s));
  }
  HIP_CHECK(hipStreamSynchronize(s));
  double total = 0;
  for (int i = 0; i < iters; i++) {
    float ms;
    HIP_CHECK(hipEventElapsedTime(&ms, ev[2 * i], ev[2 * i + 1]));
    total += ms;
  }
  for (auto& e : ev) HIP_CHECK(hipEventDestroy(e));
  return total / iters * 1e3;
}

}  // namespace

extern "C" int strasgpt_kbench_gemv_variants(void) { return sg::gemv_variant_count(); }
extern "C" int strasgpt_kbench_gemm_variants(void) { return sg::gemm_variant_count(); }

extern "C" int strasgpt_kbench_gemv(int n, int k, int dual, int variant, int iters,
                                    double* avg_us, double* rel_err) {
  if (n <= 0 || k <= 0 || k % 8 || k > 16384 || iters <= 0 || variant < 0 ||
      variant >= sg::gemv_variant_count())
    return -1;
  hipStream_t s;
  HIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  uint16_t *w, *w2 = nullptr;
  float *x, *y, *yr;
  HIP_CHECK(hipMalloc(&w, (size_t)n * k * 2));
  if (dual) HIP_CHECK(hipMalloc(&w2, (size_t)n * k * 2));
  HIP_CHECK(hipMalloc(&x, (size_t)k * 4));
  HIP_CHECK(hipMalloc(&y, (size_t)n * 4));
  HIP_CHECK(hipMalloc(&yr, (size_t)n * 4));
  hipLaunchKernelGGL(fill_bf16, dim3(1024), dim3(256), 0, s, w, (size_t)n * k, 1u);
  if (dual) hipLaunchKernelGGL(fill_bf16, dim3(1024), dim3(256), 0, s, w2, (size_t)n * k, 2u);
  hipLaunchKernelGGL(fill_f32, dim3(64), dim3(256), 0, s, x, (size_t)k, 3u);
  sg::GemvParams p{};
  p.w = w;
  p.w2 = w2;
  p.x = x;
  p.N = n;
  p.K = k;
  p.y = y;
  *avg_us = time_launches(s, iters, [&] { sg::gemv_variant(p, dual != 0, variant, s); });
  hipLaunchKernelGGL(naive_gemv, dim3((n + 255) / 256), dim3(256), 0, s, w, w2, x, n, k, yr);
  std::vector<float> a(n), b(n);
  HIP_CHECK(hipMemcpyAsync(a.data(), y, (size_t)n * 4, hipMemcpyDeviceToHost, s));
  HIP_CHECK(hipMemcpyAsync(b.data(), yr, (size_t)n * 4, hipMemcpyDeviceToHost, s));
  HIP_CHECK(hipStreamSynchronize(s));
  *rel_err = rel_error(a, b);
  HIP_CHECK(hipFree(w));
  if (w2) HIP_CHECK(hipFree(w2));
  HIP_CHECK(hipFree(x));
  HIP_CHECK(hipFree(y));
  HIP_CHECK(hipFree(yr));
  HIP_CHECK(hipStreamDestroy(s));
  return 0;
}

extern "C" int strasgpt_kbench_gemm(int m, int n, int k, int precision, int variant, int iters,
                                    double* avg_us, double* rel_err) {
  if (m <= 0 || n <= 0 || k <= 0 || k % 32 || iters <= 0 || variant < 0 ||
      variant >= sg::gemm_variant_count() || (precision != 0 && precision != 1))
    return -1;
  hipStream_t s;
  HIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  uint16_t* w;
  float *a, *c, *cr;
  HIP_CHECK(hipMalloc(&w, (size_t)n * k * 2));
  HIP_CHECK(hipMalloc(&a, (size_t)m * k * 4));
  HIP_CHECK(hipMalloc(&c, (size_t)m * n * 4));
  HIP_CHECK(hipMalloc(&cr, (size_t)m * n * 4));
  hipLaunchKernelGGL(fill_bf16, dim3(1024), dim3(256), 0, s, w, (size_t)n * k, 5u);
  hipLaunchKernelGGL(fill_f32, dim3(1024), dim3(256), 0, s, a, (size_t)m * k, 6u);
  sg::GemmParams p{};
  p.a = a;
  p.lda = k;
  p.w = w;
  p.M = m;
  p.N = n;
  p.K = k;
  p.c = c;
  p.ldc = n;
  *avg_us = time_launches(s, iters, [&] { sg::gemm_variant(p, precision, variant, s); });
  hipLaunchKernelGGL(naive_gemm, dim3((n + 255) / 256, m), dim3(256), 0, s, a, w, m, n, k, cr);
  std::vector<float> x(m * (size_t)n), y(m * (size_t)n);
  HIP_CHECK(hipMemcpyAsync(x.data(), c, x.size() * 4, hipMemcpyDeviceToHost, s));
  HIP_CHECK(hipMemcpyAsync(y.data(), cr, y.size() * 4, hipMemcpyDeviceToHost, s));
  HIP_CHECK(hipStreamSynchronize(s));
  *rel_err = rel_error(x, y);
  HIP_CHECK(hipFree(w));
  HIP_CHECK(hipFree(a));
  HIP_CHECK(hipFree(c));
  HIP_CHECK(hipFree(cr));
  HIP_CHECK(hipStreamDestroy(s));
  return 0;
}
