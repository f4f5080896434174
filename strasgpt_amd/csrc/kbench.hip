// Kernel micro-benchmarks (include/strasgpt_kbench.h): event-timed launch
// variants of the GEMV and GEMM kernels on seeded data, each checked
// against a naive reference kernel.
#include <math.h>

#include <algorithm>
#include <vector>

#include "device_common.h"
#include "grid_sync.h"
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

// One 4-byte read per 64 KiB of [p, p + bytes).
__global__ void touch_pages(const uint32_t* p, size_t bytes, uint32_t* sink) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i * 65536 < bytes) {
    const uint32_t v = __builtin_nontemporal_load(p + i * 16384);
    if (v == 0x7fc00001u) sink[0] = v;
  }
}

// Plain copy dst = src of n float4 (the calibration kernel for HBM traffic
// counters: it reads and writes exactly 16 n bytes).
__global__ __launch_bounds__(256) void copy_probe_kernel(const float4* __restrict__ src,
                                                         float4* __restrict__ dst, size_t n) {
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (size_t)gridDim.x * blockDim.x)
    dst[i] = src[i];
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

// Average of `iters` launches timed back to back between two events.
template <typename F>
double time_batch(hipStream_t s, int iters, F launch) {
  launch();
  launch();
  hipEvent_t a, b;
  HIP_CHECK(hipEventCreate(&a));
  HIP_CHECK(hipEventCreate(&b));
  HIP_CHECK(hipEventRecord(a, s));
  for (int i = 0; i < iters; i++) launch();
  HIP_CHECK(hipEventRecord(b, s));
  HIP_CHECK(hipStreamSynchronize(s));
  float ms;
  HIP_CHECK(hipEventElapsedTime(&ms, a, b));
  HIP_CHECK(hipEventDestroy(a));
  HIP_CHECK(hipEventDestroy(b));
  return ms / iters * 1e3;
}

// Average of `iters` launches, each timed by its own event pair; `before`
// runs ahead of each pair, untimed.
template <typename B, typename F>
double time_launches(hipStream_t s, int iters, B before, F launch) {
  launch();
  launch();
  std::vector<hipEvent_t> ev(2 * iters);
  for (auto& e : ev) HIP_CHECK(hipEventCreate(&e));
  for (int i = 0; i < iters; i++) {
    before();
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

// `rounds` grid barriers; before each one every block writes `words`
// 32-bit values of its own slot (two slots per block, alternating by
// round), and after it checks every value of the next block's slot.
// MODE 0: plain stores, no fences, no check (barrier cost alone);
// MODE 1: plain stores and loads with the fenced barrier;
// MODE 2: agent-coherent stores and loads with the fence-free barrier.
template <int MODE>
__global__ __launch_bounds__(256) void barrier_bench_kernel(sg::GridSync g, int rounds,
                                                           unsigned* data, int words,
                                                           unsigned* bad) {
  const unsigned b = blockIdx.x, nb = gridDim.x;
  for (int r = 0; r < rounds; r++) {
    unsigned* mine = data + ((size_t)(r & 1) * nb + b) * words;
    for (int i = threadIdx.x; i < words; i += blockDim.x) {
      if (MODE == 2)
        sg::sync_store(mine + i, r + 1);
      else
        mine[i] = r + 1;
    }
    sg::grid_sync<MODE == 1>(g);
    if (MODE != 0) {
      const unsigned* other = data + ((size_t)(r & 1) * nb + (b + 1) % nb) * words;
      unsigned miss = 0;
      for (int i = threadIdx.x; i < words; i += blockDim.x)
        miss += (MODE == 2 ? sg::sync_load(other + i) : other[i]) != (unsigned)r + 1;
      if (miss) atomicAdd(bad, miss);
    }
  }
}

}  // namespace

extern "C" int strasgpt_kbench_barrier(int blocks, int rounds, int fence, int words,
                                       double* us_per_round, int* bad_reads, int* timed_out) {
  if (blocks <= 0 || rounds <= 0 || words <= 0 || words > 65536) return -1;
  int dev, cus, per_cu = 0;
  HIP_CHECK(hipGetDevice(&dev));
  HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  if (fence < 0 || fence > 2) return -1;
  const void* fn = fence == 0   ? (const void*)barrier_bench_kernel<0>
                   : fence == 1 ? (const void*)barrier_bench_kernel<1>
                                : (const void*)barrier_bench_kernel<2>;
  HIP_CHECK(hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, 256, 0));
  if (blocks > per_cu * cus) return -2;  // not all blocks resident at once
  hipStream_t s;
  HIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  if (blocks > sg::kSyncMaxBlocks) return -1;
  unsigned *state, *flags, *data;
  HIP_CHECK(hipMalloc(&state, sg::kSyncStateWords * 4));
  HIP_CHECK(hipMalloc(&flags, 64));
  HIP_CHECK(hipMalloc(&data, (size_t)2 * blocks * words * 4));
  HIP_CHECK(hipMemsetAsync(state, 0, sg::kSyncStateWords * 4, s));
  HIP_CHECK(hipMemsetAsync(flags, 0, 64, s));
  HIP_CHECK(hipMemsetAsync(data, 0, (size_t)2 * blocks * words * 4, s));
  sg::GridSync g{state, flags, 1u};
  unsigned* bad = flags + 1;
  void* args[] = {&g, &rounds, &data, &words, &bad};
  hipEvent_t a, b;
  HIP_CHECK(hipEventCreate(&a));
  HIP_CHECK(hipEventCreate(&b));
  HIP_CHECK(hipLaunchCooperativeKernel(fn, dim3(blocks), dim3(256), args, 0, s));  // warm-up
  g.seq += rounds;
  HIP_CHECK(hipEventRecord(a, s));
  HIP_CHECK(hipLaunchCooperativeKernel(fn, dim3(blocks), dim3(256), args, 0, s));
  HIP_CHECK(hipEventRecord(b, s));
  HIP_CHECK(hipStreamSynchronize(s));
  float ms;
  HIP_CHECK(hipEventElapsedTime(&ms, a, b));
  *us_per_round = ms * 1e3 / rounds;
  unsigned h[2];
  HIP_CHECK(hipMemcpy(h, flags, 8, hipMemcpyDeviceToHost));
  *timed_out = (int)h[0];
  *bad_reads = (int)h[1];
  HIP_CHECK(hipEventDestroy(a));
  HIP_CHECK(hipEventDestroy(b));
  HIP_CHECK(hipFree(state));
  HIP_CHECK(hipFree(flags));
  HIP_CHECK(hipFree(data));
  HIP_CHECK(hipStreamDestroy(s));
  return 0;
}

extern "C" int strasgpt_kbench_copy(size_t bytes, int iters, double* avg_us) {
  if (bytes < 16 || bytes % 16 || iters <= 0) return -1;
  hipStream_t s;
  HIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  float4 *a, *b;
  HIP_CHECK(hipMalloc(&a, bytes));
  HIP_CHECK(hipMalloc(&b, bytes));
  hipLaunchKernelGGL(fill_f32, dim3(1024), dim3(256), 0, s, (float*)a, bytes / 4, 7u);
  const size_t n = bytes / 16;
  *avg_us = time_launches(s, iters, [] {}, [&] {
    hipLaunchKernelGGL(copy_probe_kernel, dim3(2048), dim3(256), 0, s, a, b, n);
  });
  HIP_CHECK(hipStreamSynchronize(s));
  HIP_CHECK(hipFree(a));
  HIP_CHECK(hipFree(b));
  HIP_CHECK(hipStreamDestroy(s));
  return 0;
}

extern "C" int strasgpt_kbench_mxfp4_decode(const uint8_t* codes, const uint8_t* scales, int nblocks,
                                            float* out) {
  if (nblocks <= 0) return -1;
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

extern "C" int strasgpt_kbench_gemv_variants(void) { return sg::gemv_variant_count(); }
extern "C" int strasgpt_kbench_gemm_variants(void) { return sg::gemm_variant_count(); }

extern "C" int strasgpt_kbench_gemv(int n, int k, int dual, int variant, int iters,
                                    double* avg_us, double* rel_err) {
  return strasgpt_kbench_gemv2(n, k, dual, 0, variant, iters, avg_us, rel_err);
}

extern "C" int strasgpt_kbench_gemv2(int n, int k, int dual, int flags, int variant, int iters,
                                     double* avg_us, double* rel_err) {
  const bool norm = flags & 1, touch = flags & 2, batch = flags & 4, reuse = flags & 8;
  if (n <= 0 || k <= 0 || k % 8 || k > 16384 || iters <= 0 || variant < 0 ||
      variant >= sg::gemv_variant_count())
    return -1;
  hipStream_t s;
  HIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  // Enough distinct weight copies to exceed the 256 MiB Infinity Cache
  // twice over, used round-robin so that every launch streams from HBM
  // (flag 8: one copy, re-read by every launch).
  const size_t bytes = (size_t)n * k * 2 * (dual ? 2 : 1);
  const int copies =
      reuse ? 1 : (int)std::min<size_t>(64, std::max<size_t>(2, (size_t)(1u << 30) / bytes + 1));
  std::vector<uint16_t*> w(copies), w2(copies, nullptr);
  uint16_t* nw = nullptr;
  float *x, *y, *yr, *xn;
  uint32_t* sink;
  HIP_CHECK(hipMalloc(&sink, 4));
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
  const size_t mat = (size_t)n * k * 2, pages = (mat + 65535) / 65536;
  auto run = [&] {
    p.w = w[it % copies];
    p.w2 = w2[it % copies];
    it++;
    sg::gemv_variant(p, dual != 0, variant, s);
  };
  auto warm = [&] {
    if (!touch) return;
    const int c = it % copies;
    hipLaunchKernelGGL(touch_pages, dim3((pages + 255) / 256), dim3(256), 0, s,
                       (const uint32_t*)w[c], mat, sink);
    if (dual)
      hipLaunchKernelGGL(touch_pages, dim3((pages + 255) / 256), dim3(256), 0, s,
                         (const uint32_t*)w2[c], mat, sink);
  };
  *avg_us = batch ? time_batch(s, iters, run) : time_launches(s, iters, warm, run);
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
  HIP_CHECK(hipFree(sink));
  HIP_CHECK(hipStreamDestroy(s));
  return 0;
}

extern "C" int strasgpt_kbench_gemm(int m, int n, int k, int precision, int variant, int iters,
                                    double* avg_us, double* rel_err) {
  if (m <= 0 || n <= 0 || k <= 0 || k % 32 || iters <= 0 || variant < 0 ||
      variant >= sg::gemm_variant_count() || (precision & ~3))
    return -1;
  // precision bit 1: evict the caches (write 512 MiB) before each timed
  // launch, so the weights come from HBM as in a prefill pass.
  const bool cold = precision & 2;
  precision &= 1;
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
  void* flush = nullptr;
  const size_t flush_bytes = (size_t)512 << 20;
  if (cold) HIP_CHECK(hipMalloc(&flush, flush_bytes));
  *avg_us = time_launches(
      s, iters,
      [&] {
        if (cold) HIP_CHECK(hipMemsetAsync(flush, 0, flush_bytes, s));
      },
      [&] { sg::gemm_variant(p, precision, variant, s); });
  if (flush) HIP_CHECK(hipFree(flush));
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

extern "C" int strasgpt_kbench_attn_prefill(int T, int P, int q_heads, int kv_heads, int hd, int variant,
                                            int iters, double* avg_us) {
  if (T <= 0 || P < 0 || q_heads <= 0 || kv_heads <= 0 || q_heads % kv_heads || iters <= 0 ||
      (hd != 16 && hd != 32 && hd != 64 && hd != 128) || (variant != 0 && variant != 1))
    return -1;
  hipStream_t s;
  HIP_CHECK(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
  const int ctx = P + T;
  float *q, *kc, *vc;
  uint16_t *hi, *lo;
  int* pos;
  const size_t nq = (size_t)T * q_heads * hd, nkv = (size_t)kv_heads * ctx * hd;
  HIP_CHECK(hipMalloc(&q, nq * 4));
  HIP_CHECK(hipMalloc(&kc, nkv * 4));
  HIP_CHECK(hipMalloc(&vc, nkv * 4));
  HIP_CHECK(hipMalloc(&hi, nq * 2));
  HIP_CHECK(hipMalloc(&lo, nq * 2));
  HIP_CHECK(hipMalloc(&pos, sizeof(int)));
  hipLaunchKernelGGL(fill_f32, dim3(1024), dim3(256), 0, s, q, nq, 11u);
  hipLaunchKernelGGL(fill_f32, dim3(1024), dim3(256), 0, s, kc, nkv, 12u);
  hipLaunchKernelGGL(fill_f32, dim3(1024), dim3(256), 0, s, vc, nkv, 13u);
  HIP_CHECK(hipMemcpyAsync(pos, &P, sizeof(int), hipMemcpyHostToDevice, s));
  const int ctx_pad = (ctx + 31) / 32 * 32;
  uint16_t *khi, *klo, *vhi, *vlo;
  const size_t nvt = (size_t)kv_heads * hd * ctx_pad;
  HIP_CHECK(hipMalloc(&khi, nkv * 2));
  HIP_CHECK(hipMalloc(&klo, nkv * 2));
  HIP_CHECK(hipMalloc(&vhi, nvt * 2));
  HIP_CHECK(hipMalloc(&vlo, nvt * 2));
  HIP_CHECK(hipMemsetAsync(vhi, 0, nvt * 2, s));
  HIP_CHECK(hipMemsetAsync(vlo, 0, nvt * 2, s));
  sg::attention_split_rows(kc, vc, khi, klo, vhi, vlo, kv_heads, ctx, ctx_pad, hd, 0, ctx, s);
  sg::AttnParams p{};
  p.q = q;
  p.kcache = kc;
  p.vcache = vc;
  p.khi = khi;
  p.klo = klo;
  p.vthi = vhi;
  p.vtlo = vlo;
  p.ctx_pad = ctx_pad;
  p.out_hi = hi;
  p.out_lo = lo;
  p.pos = pos;
  p.T = T;
  p.q_heads = q_heads;
  p.kv_heads = kv_heads;
  p.hd = hd;
  p.ctx = ctx;
  p.q0 = 0;
  *avg_us = time_launches(s, iters, [] {}, [&] { sg::attention_prefill_variant(p, variant, s); });
  HIP_CHECK(hipStreamSynchronize(s));
  HIP_CHECK(hipFree(q));
  HIP_CHECK(hipFree(kc));
  HIP_CHECK(hipFree(vc));
  HIP_CHECK(hipFree(hi));
  HIP_CHECK(hipFree(lo));
  HIP_CHECK(hipFree(pos));
  HIP_CHECK(hipFree(khi));
  HIP_CHECK(hipFree(klo));
  HIP_CHECK(hipFree(vhi));
  HIP_CHECK(hipFree(vlo));
  HIP_CHECK(hipStreamDestroy(s));
  return 0;
}
