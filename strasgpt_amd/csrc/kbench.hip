// Kernel micro-benchmarks (include/strasgpt_kbench.h): event-timed launch
// variants of the GEMV and GEMM kernels on seeded data, each checked
// against a naive reference kernel.
#include <math.h>

#include <algorithm>
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

__global__ void split_planes(const float* a, size_t n, uint16_t* hi, uint16_t* lo) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    const uint16_t h = f32_to_bf16_rne(a[i]);
    hi[i] = h;
    lo[i] = f32_to_bf16_rne(a[i] - bf16_to_f32(h));
  }
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
  return strasgpt_kbench_gemv2(n, k, dual, 0, variant, iters, avg_us, rel_err);
}

extern "C" int strasgpt_kbench_gemv2(int n, int k, int dual, int norm, int variant, int iters,
                                     double* avg_us, double* rel_err) {
  if (n <= 0 || k <= 0 || k % 8 || k > 16384 || iters <= 0 || variant < 0 ||
      variant >= sg::gemv_variant_count())
    return -1;
  hipStream_t s;
  HIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  // Enough distinct weight copies to exceed the 256 MiB Infinity Cache
  // twice over, used round-robin so that every launch streams from HBM.
  const size_t bytes = (size_t)n * k * 2 * (dual ? 2 : 1);
  const int copies = (int)std::min<size_t>(64, std::max<size_t>(2, (size_t)(1u << 30) / bytes + 1));
  std::vector<uint16_t*> w(copies), w2(copies, nullptr);
  uint16_t* nw = nullptr;
  float *x, *y, *yr, *xn;
  for (int c = 0; c < copies; c++) {
    HIP_CHECK(hipMalloc(&w[c], (size_t)n * k * 2));
    hipLaunchKernelGGL(fill_bf16, dim3(1024), dim3(256), 0, s, w[c], (size_t)n * k, 1u);
    if (dual) {
      HIP_CHECK(hipMalloc(&w2[c], (size_t)n * k * 2));
      hipLaunchKernelGGL(fill_bf16, dim3(1024), dim3(256), 0, s, w2[c], (size_t)n * k, 2u);
    }
  }
  HIP_CHECK(hipMalloc(&x, (size_t)k * 4));
  HIP_CHECK(hipMalloc(&xn, (size_t)k * 4));
  HIP_CHECK(hipMalloc(&y, (size_t)n * 4));
  HIP_CHECK(hipMalloc(&yr, (size_t)n * 4));
  hipLaunchKernelGGL(fill_f32, dim3(64), dim3(256), 0, s, x, (size_t)k, 3u);
  if (norm) {
    HIP_CHECK(hipMalloc(&nw, (size_t)k * 2));
    hipLaunchKernelGGL(fill_bf16, dim3(64), dim3(256), 0, s, nw, (size_t)k, 4u);
  }
  sg::GemvParams p{};
  p.x = x;
  p.norm_w = nw;
  p.eps = 1e-6f;
  p.N = n;
  p.K = k;
  p.y = y;
  int it = 0;
  *avg_us = time_launches(s, iters, [&] {
    p.w = w[it % copies];
    p.w2 = w2[it % copies];
    it++;
    sg::gemv_variant(p, dual != 0, variant, s);
  });
  // reference on the last matrix used
  const float* xin = x;
  if (norm) {
    sg::rmsnorm_rows(x, nw, xn, 1, k, 1e-6f, s);
    xin = xn;
  }
  hipLaunchKernelGGL(naive_gemv, dim3((n + 255) / 256), dim3(256), 0, s, p.w, p.w2, xin, n, k, yr);
  std::vector<float> a(n), b(n);
  HIP_CHECK(hipMemcpyAsync(a.data(), y, (size_t)n * 4, hipMemcpyDeviceToHost, s));
  HIP_CHECK(hipMemcpyAsync(b.data(), yr, (size_t)n * 4, hipMemcpyDeviceToHost, s));
  HIP_CHECK(hipStreamSynchronize(s));
  *rel_err = rel_error(a, b);
  for (int c = 0; c < copies; c++) {
    HIP_CHECK(hipFree(w[c]));
    if (w2[c]) HIP_CHECK(hipFree(w2[c]));
  }
  if (nw) HIP_CHECK(hipFree(nw));
  HIP_CHECK(hipFree(x));
  HIP_CHECK(hipFree(xn));
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
  uint16_t *w, *ahi, *alo;
  float *a, *c, *cr;
  HIP_CHECK(hipMalloc(&w, (size_t)n * k * 2));
  HIP_CHECK(hipMalloc(&a, (size_t)m * k * 4));
  HIP_CHECK(hipMalloc(&ahi, (size_t)m * k * 2));
  HIP_CHECK(hipMalloc(&alo, (size_t)m * k * 2));
  HIP_CHECK(hipMalloc(&c, (size_t)m * n * 4));
  HIP_CHECK(hipMalloc(&cr, (size_t)m * n * 4));
  hipLaunchKernelGGL(fill_bf16, dim3(1024), dim3(256), 0, s, w, (size_t)n * k, 5u);
  hipLaunchKernelGGL(fill_f32, dim3(1024), dim3(256), 0, s, a, (size_t)m * k, 6u);
  hipLaunchKernelGGL(split_planes, dim3(1024), dim3(256), 0, s, a, (size_t)m * k, ahi, alo);
  sg::GemmParams p{};
  p.a_hi = ahi;
  p.a_lo = alo;
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
  HIP_CHECK(hipFree(ahi));
  HIP_CHECK(hipFree(alo));
  HIP_CHECK(hipFree(c));
  HIP_CHECK(hipFree(cr));
  HIP_CHECK(hipStreamDestroy(s));
  return 0;
}
