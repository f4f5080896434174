// Decode GEMV on gfx950: one fp32 activation row against bf16 [N][K]
// weights streamed from HBM once per step.
//
// Mapping: a 256-thread block (4 wavefronts) stages the input row, RMSNorm
// applied when requested, in LDS as fp32; each wavefront owns R output
// rows at a time and walks K with 128-bit non-temporal loads (8 bf16 per
// lane, 512 elements per wavefront per step), four K steps in flight per
// row. The bf16 -> fp32 conversion is a shift in registers (exact), the
// products are fp32 FMAs, and the row sum is a 64-lane reduction. Blocks
// stride over row groups (a persistent grid of at most 8 blocks per CU) so
// the staged row is reused across many weight rows.
//
// Algorithmic bytes per launch: N * K * 2 (x2 for the SwiGLU pair).
#include "device_common.h"
#include "hip_check.h"
#include "kernels.h"

namespace sg {

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / WAVE;
constexpr int kMaxLdsK = 16384;  // fp32 row staged in LDS up to 64 KiB

__device__ __forceinline__ float dot8(uint4 w, const float4& a, const float4& b, float acc) {
  acc = fmaf(bf16_lo(w.x), a.x, acc);
  acc = fmaf(bf16_hi(w.x), a.y, acc);
  acc = fmaf(bf16_lo(w.y), a.z, acc);
  acc = fmaf(bf16_hi(w.y), a.w, acc);
  acc = fmaf(bf16_lo(w.z), b.x, acc);
  acc = fmaf(bf16_hi(w.z), b.y, acc);
  acc = fmaf(bf16_lo(w.w), b.z, acc);
  acc = fmaf(bf16_hi(w.w), b.w, acc);
  return acc;
}

__device__ __forceinline__ float silu_mul(float g, float u) {
  // reference source/transformer.c:1477-1486
  g *= 1.0f / (1.0f + expf(-g));
  return g * u;
}

template <bool NORM, bool LDS>
__device__ __forceinline__ void stage_row(const GemvParams& p, float* xs, float* red) {
  const int K = p.K;
  if (!LDS) return;
  if (NORM) {
    float ss = 0.0f;
    for (int k = threadIdx.x * 4; k < K; k += kThreads * 4) {
      float4 v = *(const float4*)(p.x + k);
      ss = fmaf(v.x, v.x, ss);
      ss = fmaf(v.y, v.y, ss);
      ss = fmaf(v.z, v.z, ss);
      ss = fmaf(v.w, v.w, ss);
    }
    const float s = rms_scale(block_sum<kThreads>(ss, red), K, p.eps);
    for (int k = threadIdx.x; k < K; k += kThreads)
      xs[k] = (p.x[k] * s) * bf16_to_f32(p.norm_w[k]);
  } else {
    for (int k = threadIdx.x * 4; k < K; k += kThreads * 4)
      *(float4*)(xs + k) = *(const float4*)(p.x + k);
  }
  __syncthreads();
}

template <int R, int EPI, bool NORM, bool LDS>
__global__ __launch_bounds__(kThreads) void gemv_kernel(GemvParams p) {
  extern __shared__ float xs[];
  __shared__ float red[kWaves];
  stage_row<NORM, LDS>(p, xs, red);
  const float* xr = LDS ? xs : p.x;

  const int lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  const int K = p.K, N = p.N;
  constexpr bool DUAL = EPI == GEMV_SWIGLU;
  const int stride = gridDim.x * kWaves * R;

  for (int row0 = (blockIdx.x * kWaves + wave) * R; row0 < N; row0 += stride) {
    float acc[R], acc2[R];
    const uint16_t* wr[R];
    const uint16_t* wr2[R];
#pragma unroll
    for (int r = 0; r < R; r++) {
      acc[r] = 0.0f;
      acc2[r] = 0.0f;
      const int row = min(row0 + r, N - 1);  // clamp: tail rows recompute row N-1
      wr[r] = p.w + (size_t)row * K;
      wr2[r] = DUAL ? p.w2 + (size_t)row * K : nullptr;
    }
    int k = lane * 8;
    // Four K steps per row in flight.
    for (; k + 3 * 512 < K; k += 4 * 512) {
      uint4 wv[4][R], wv2[4][R];
#pragma unroll
      for (int u = 0; u < 4; u++)
#pragma unroll
        for (int r = 0; r < R; r++) {
          wv[u][r] = load_nt_u4(wr[r] + k + u * 512);
          if (DUAL) wv2[u][r] = load_nt_u4(wr2[r] + k + u * 512);
        }
#pragma unroll
      for (int u = 0; u < 4; u++) {
        const float4 a = *(const float4*)(xr + k + u * 512);
        const float4 b = *(const float4*)(xr + k + u * 512 + 4);
#pragma unroll
        for (int r = 0; r < R; r++) {
          acc[r] = dot8(wv[u][r], a, b, acc[r]);
          if (DUAL) acc2[r] = dot8(wv2[u][r], a, b, acc2[r]);
        }
      }
    }
    for (; k < K; k += 512) {
      const float4 a = *(const float4*)(xr + k);
      const float4 b = *(const float4*)(xr + k + 4);
#pragma unroll
      for (int r = 0; r < R; r++) {
        acc[r] = dot8(load_nt_u4(wr[r] + k), a, b, acc[r]);
        if (DUAL) acc2[r] = dot8(load_nt_u4(wr2[r] + k), a, b, acc2[r]);
      }
    }
#pragma unroll
    for (int r = 0; r < R; r++) {
      acc[r] = wave_sum(acc[r]);
      if (DUAL) acc2[r] = wave_sum(acc2[r]);
    }
    if (lane == 0) {
#pragma unroll
      for (int r = 0; r < R; r++) {
        const int n = row0 + r;
        if (n >= N) break;
        if (EPI == GEMV_STORE) {
          p.y[n] = acc[r];
        } else if (EPI == GEMV_RESIDUAL) {
          p.y[n] += acc[r];
        } else if (EPI == GEMV_SWIGLU) {
          p.y[n] = silu_mul(acc[r], acc2[r]);
        } else {  // GEMV_QKV
          if (n < p.q_dim) {
            p.q[n] = acc[r];
          } else if (n < p.q_dim + p.kv_dim) {
            p.kraw[n - p.q_dim] = acc[r];
          } else {
            const int j = n - p.q_dim - p.kv_dim;
            const int head = j / p.head_dim, h = j % p.head_dim;
            p.vcache[((size_t)head * p.ctx + *p.pos) * p.head_dim + h] = acc[r];
          }
        }
      }
    }
  }
}

template <int R, int EPI>
void launch(const GemvParams& p, hipStream_t s) {
  const bool lds = p.K <= kMaxLdsK;
  const int rows_per_block = kWaves * R;
  int blocks = (p.N + rows_per_block - 1) / rows_per_block;
  blocks = blocks < 2048 ? blocks : 2048;
  const size_t shm = lds ? (size_t)p.K * sizeof(float) : 0;
  if (p.norm_w) {
    if (!lds) ST_DIE("GEMV with RMSNorm needs K <= 16384");
    hipLaunchKernelGGL((gemv_kernel<R, EPI, true, true>), dim3(blocks), dim3(kThreads), shm, s, p);
  } else if (lds) {
    hipLaunchKernelGGL((gemv_kernel<R, EPI, false, true>), dim3(blocks), dim3(kThreads), shm, s, p);
  } else {
    hipLaunchKernelGGL((gemv_kernel<R, EPI, false, false>), dim3(blocks), dim3(kThreads), 0, s, p);
  }
}

}  // namespace

void gemv(const GemvParams& p, int epi, hipStream_t s) {
  if (p.K <= 0 || p.K % 8 != 0) ST_DIE("GEMV needs K to be a positive multiple of 8");
  if (p.N <= 0) ST_DIE("GEMV needs N > 0");
  if (((uintptr_t)p.w | (uintptr_t)p.x) % 16 != 0) ST_DIE("GEMV operands must be 16-byte aligned");
  if (epi == GEMV_SWIGLU && (!p.w2 || (uintptr_t)p.w2 % 16)) ST_DIE("GEMV SwiGLU needs an aligned up matrix");
  if (epi == GEMV_QKV && p.N != p.q_dim + 2 * p.kv_dim) ST_DIE("GEMV QKV row count mismatch");
  switch (epi) {
    case GEMV_STORE: launch<2, GEMV_STORE>(p, s); break;
    case GEMV_RESIDUAL: launch<1, GEMV_RESIDUAL>(p, s); break;
    case GEMV_QKV: launch<2, GEMV_QKV>(p, s); break;
    case GEMV_SWIGLU: launch<1, GEMV_SWIGLU>(p, s); break;
    default: ST_DIE("unknown GEMV epilogue");
  }
  HIP_CHECK(hipGetLastError());
}

}  // namespace sg
