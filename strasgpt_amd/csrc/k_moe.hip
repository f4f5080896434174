// Mixture-of-experts FFN kernels (no reference counterpart; semantics are
// defined by this library and restated by the CPU oracle):
//   router   logits_e = W_r[e] . xn (bf16 weights, fp32 accumulate),
//            the k largest in descending order (ties: lowest expert id),
//            weights = softmax over those k logits;
//   experts  a_j = silu(G_e xn) * (U_e xn) with MXFP4 G_e, U_e;
//            out = sum_j w_j (D_e a_j), accumulated in top-k order as
//            acc = fmaf(w_j, D_e a_j, acc), then x += acc.
// MXFP4 rows are [K/32] blocks of 16 code bytes (element 2i in the low
// nibble) and one E8M0 exponent each: one 128-bit load per lane covers a
// whole 32-value block, decoded in registers (exact in fp32).
#include "device_common.h"
#include "hip_check.h"
#include "kernels.h"

namespace sg {

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / WAVE;
constexpr int kRowsPerWave = 4;

// Dot of one MXFP4 row with an fp32 vector in LDS (K multiple of 32).
__device__ __forceinline__ float mx_row_dot(const uint8_t* blocks, const uint8_t* scales,
                                            const float* xs, int K, int lane) {
  float acc = 0.0f;
  const int nb = K / 32;
  for (int b = lane; b < nb; b += WAVE) {
    const uint4 q = load_nt_u4(blocks + (size_t)b * 16);
    const float sc = e8m0_scale(scales[b]);
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
    const float* xb = xs + b * 32;
#pragma unroll
    for (int i = 0; i < 4; i++) {
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const uint32_t byte = (w[i] >> (8 * j)) & 0xFFu;
        const int e = (i * 4 + j) * 2;
        acc = fmaf(e2m1_value(byte & 15u) * sc, xb[e], acc);
        acc = fmaf(e2m1_value(byte >> 4) * sc, xb[e + 1], acc);
      }
    }
  }
  return wave_sum(acc);
}

// Router + top-k + softmax, one block per token.
__global__ __launch_bounds__(kThreads) void route_kernel(const float* xn, const uint16_t* router,
                                                         int E, int d, int k, int* sel,
                                                         float* sel_w) {
  extern __shared__ float sm[];
  float* xs = sm;        // [d]
  float* lg = sm + d;    // [E]
  const int t = blockIdx.x, lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  for (int i = threadIdx.x; i < d; i += kThreads) xs[i] = xn[(size_t)t * d + i];
  __syncthreads();
  for (int e = wave; e < E; e += kWaves) {
    const uint16_t* wr = router + (size_t)e * d;
    float acc = 0.0f;
    for (int i = lane; i < d; i += WAVE) acc = fmaf(bf16_to_f32(wr[i]), xs[i], acc);
    acc = wave_sum(acc);
    if (lane == 0) lg[e] = acc;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int idx[64];
    float val[64];
    for (int j = 0; j < k; j++) {
      int best = -1;
      for (int e = 0; e < E; e++) {
        bool taken = false;
        for (int q = 0; q < j; q++) taken |= idx[q] == e;
        if (taken) continue;
        if (best < 0 || lg[e] > lg[best]) best = e;
      }
      idx[j] = best;
      val[j] = lg[best];
    }
    float sum = 0.0f;
    for (int j = 0; j < k; j++) {
      val[j] = expf(val[j] - lg[idx[0]]);
      sum += val[j];
    }
    for (int j = 0; j < k; j++) {
      sel[t * k + j] = idx[j];
      sel_w[t * k + j] = val[j] / sum;
    }
  }
}

// act[s][h] = silu(gate_e[h] . x_s) * (up_e[h] . x_s), slot s = (token, j).
__global__ __launch_bounds__(kThreads) void swiglu_kernel(MoeGemvParams p) {
  extern __shared__ float xs[];
  const int slot = blockIdx.y, lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  const float* xr = p.x + (size_t)(slot / p.topk) * p.K;
  for (int i = threadIdx.x; i < p.K; i += kThreads) xs[i] = xr[i];
  __syncthreads();
  const int e = p.expert[slot];
  const size_t rb = (size_t)p.K / 2, rs = (size_t)p.K / 32;
  const int r0 = (blockIdx.x * kWaves + wave) * kRowsPerWave;
  for (int r = r0; r < min(r0 + kRowsPerWave, p.N); r++) {
    const size_t row = (size_t)e * p.N + r;
    const float g = mx_row_dot(p.blocks + row * rb, p.scales + row * rs, xs, p.K, lane);
    const float u = mx_row_dot(p.blocks2 + row * rb, p.scales2 + row * rs, xs, p.K, lane);
    if (lane == 0) p.y[(size_t)slot * p.N + r] = silu_mul(g, u);
  }
}

// y[t][n] += sum_j fmaf order of w_j * (down_e_j[n] . act[t*k + j]).
__global__ __launch_bounds__(kThreads) void down_kernel(MoeGemvParams p) {
  extern __shared__ float as[];  // [k][K]
  const int k = p.topk;
  const int t = blockIdx.y, lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  for (int i = threadIdx.x; i < k * p.K; i += kThreads) as[i] = p.x[(size_t)t * k * p.K + i];
  __syncthreads();
  const size_t rb = (size_t)p.K / 2, rs = (size_t)p.K / 32;
  const int r0 = (blockIdx.x * kWaves + wave) * kRowsPerWave;
  for (int r = r0; r < min(r0 + kRowsPerWave, p.N); r++) {
    float acc = 0.0f;
    for (int j = 0; j < k; j++) {
      const int e = p.expert[t * k + j];
      const size_t row = (size_t)e * p.N + r;
      const float v = mx_row_dot(p.blocks + row * rb, p.scales + row * rs, as + j * p.K, p.K, lane);
      acc = fmaf(p.weight[t * k + j], v, acc);
    }
    if (lane == 0) p.y[(size_t)t * p.N + r] += acc;
  }
}

template <typename F>
void set_lds(F kernel, size_t bytes) {
  if (bytes > 160 * 1024) ST_DIE("MoE kernel rows do not fit in LDS");
  if (bytes > 64 * 1024)
    HIP_CHECK(hipFuncSetAttribute((const void*)kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                  (int)bytes));
}

}  // namespace

void moe_route(const float* xn, int T, const uint16_t* router, int E, int d, int k, int* sel,
               float* sel_w, hipStream_t s) {
  if (k > 64 || k > E || E > 1024) ST_DIE("MoE top-k must satisfy k <= 64, k <= E <= 1024");
  const size_t shm = (size_t)(d + E) * sizeof(float);
  set_lds(route_kernel, shm);
  hipLaunchKernelGGL(route_kernel, dim3(T), dim3(kThreads), shm, s, xn, router, E, d, k, sel, sel_w);
  HIP_CHECK(hipGetLastError());
}

void moe_gemv_swiglu(const MoeGemvParams& p, hipStream_t s) {
  if (p.K % 32 || ((uintptr_t)p.blocks | (uintptr_t)p.blocks2) % 16) ST_DIE("MXFP4 rows must be 32-value aligned");
  if (p.topk <= 0 || p.tokens <= 0) ST_DIE("MoE GEMV needs tokens and topk");
  const size_t shm = (size_t)p.K * sizeof(float);
  set_lds(swiglu_kernel, shm);
  const int rows_per_block = kWaves * kRowsPerWave;
  dim3 grid((p.N + rows_per_block - 1) / rows_per_block, p.tokens * p.topk);
  hipLaunchKernelGGL(swiglu_kernel, grid, dim3(kThreads), shm, s, p);
  HIP_CHECK(hipGetLastError());
}

void moe_gemv_down(const MoeGemvParams& p, hipStream_t s) {
  if (p.K % 32 || (uintptr_t)p.blocks % 16) ST_DIE("MXFP4 rows must be 32-value aligned");
  if (p.topk <= 0 || p.tokens <= 0) ST_DIE("MoE GEMV needs tokens and topk");
  const size_t shm = (size_t)p.topk * p.K * sizeof(float);
  set_lds(down_kernel, shm);
  const int rows_per_block = kWaves * kRowsPerWave;
  dim3 grid((p.N + rows_per_block - 1) / rows_per_block, p.tokens);
  hipLaunchKernelGGL(down_kernel, grid, dim3(kThreads), shm, s, p);
  HIP_CHECK(hipGetLastError());
}

}  // namespace sg
