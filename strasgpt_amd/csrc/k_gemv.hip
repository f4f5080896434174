// Decode GEMV on gfx950: one fp32 activation row against bf16 [N][K]
// weights streamed from HBM once per step.
//
// Mapping: a 256-thread block (4 wavefronts) stages the input row, RMSNorm
// applied when requested, in LDS as fp32; each wavefront owns R output
// rows at a time and walks K with 128-bit non-temporal loads (8 bf16 per
// lane, 512 elements per wavefront per step). Weight loads are issued in
// chunks of U steps, double-buffered in registers: the first chunk is in
// flight before the block stages the input row, and chunk c+1 is in flight
// while chunk c is multiplied. The bf16 -> fp32 conversion is a shift in
// registers (exact), the products are fp32 FMAs, and each row ends with a
// 64-lane reduction. The grid is sized so that every block handles the
// same number of row groups.
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
constexpr int kStep = 8 * WAVE;  // K elements per wavefront step
constexpr int kXcds = 8;

template <bool NORM>
__device__ __forceinline__ void stage_row(const GemvParams& p, float* xs, float* red) {
  const int K = p.K;
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

template <int R, int U, bool DUAL>
struct Chunk {
  uint4 w[U][R];
  uint4 w2[DUAL ? U : 1][DUAL ? R : 1];
};

// Loads chunk c (U steps of 512 elements) of rows row0..row0+R-1; steps
// beyond K are not loaded (their registers are never read).
template <int R, int U, bool DUAL>
__device__ __forceinline__ void load_chunk(const GemvParams& p, int row0, int c, int lane,
                                           Chunk<R, U, DUAL>& ch) {
  const int N = p.N, K = p.K;
#pragma unroll
  for (int r = 0; r < R; r++) {
    const int row = min(row0 + r, N - 1);  // tail rows recompute row N-1, never stored
    const uint16_t* wr = p.w + (size_t)row * K;
    const uint16_t* wr2 = DUAL ? p.w2 + (size_t)row * K : nullptr;
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int k = (c * U + u) * kStep + lane * 8;
      if (k < K) {
        ch.w[u][r] = load_nt_u4(wr + k);
        if (DUAL) ch.w2[u][r] = load_nt_u4(wr2 + k);
      }
    }
  }
}

template <int R, int U, bool DUAL>
__device__ __forceinline__ void mul_chunk(const float* xr, int K, int c, int lane,
                                          const Chunk<R, U, DUAL>& ch, float* acc, float* acc2) {
#pragma unroll
  for (int u = 0; u < U; u++) {
    const int k = (c * U + u) * kStep + lane * 8;
    if (k < K) {
      const float4 a = *(const float4*)(xr + k);
      const float4 b = *(const float4*)(xr + k + 4);
#pragma unroll
      for (int r = 0; r < R; r++) {
        acc[r] = dot8(ch.w[u][r], a, b, acc[r]);
        if (DUAL) acc2[r] = dot8(ch.w2[u][r], a, b, acc2[r]);
      }
    }
  }
}

template <int R, int U, int EPI, bool NORM, bool LDS>
__global__ __launch_bounds__(kThreads) void gemv_kernel(GemvParams p) {
  extern __shared__ float xs[];
  __shared__ float red[kWaves];
  constexpr bool DUAL = EPI == GEMV_SWIGLU;
  const int lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  const int K = p.K, N = p.N;
  const int nchunks = (K + U * kStep - 1) / (U * kStep);
  // Each block owns a contiguous range of row groups. Blocks are dispatched
  // round-robin over the 8 XCDs; renumbering gives every XCD a contiguous
  // slice of the matrix, so each XCD's TLB and L2 see 1/8 of its pages.
  const int groups = (N + kWaves * R - 1) / (kWaves * R);
  const int G = gridDim.x, per = (groups + G - 1) / G;
  const int v = (G % kXcds == 0) ? (blockIdx.x % kXcds) * (G / kXcds) + blockIdx.x / kXcds
                                 : blockIdx.x;
  const int g_end = min(groups, (v + 1) * per);
  const int stride = kWaves * R;  // rows per group
  int row0 = (v * per * kWaves + wave) * R;
  const int row_end = g_end * kWaves * R;

  Chunk<R, U, DUAL> cur, nxt;
  if (row0 < min(N, row_end)) load_chunk<R, U, DUAL>(p, row0, 0, lane, cur);
  if (LDS) stage_row<NORM>(p, xs, red);
  const float* xr = LDS ? xs : p.x;

  for (; row0 < min(N, row_end); row0 += stride) {
    float acc[R], acc2[R];
#pragma unroll
    for (int r = 0; r < R; r++) acc[r] = acc2[r] = 0.0f;
    for (int c = 0; c < nchunks; c++) {
      // Issue the next chunk (of this row group, or the first chunk of the
      // next one) before multiplying the current one.
      const bool more = c + 1 < nchunks;
      const int nrow = more ? row0 : row0 + stride;
      if (more || nrow < min(N, row_end)) load_chunk<R, U, DUAL>(p, nrow, more ? c + 1 : 0, lane, nxt);
      mul_chunk<R, U, DUAL>(xr, K, c, lane, cur, acc, acc2);
      cur = nxt;
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

// Blocks: at most `cap`, the same number of row groups for each block, and
// a multiple of the XCD count when there are enough groups.
int balanced_blocks(int groups, int cap) {
  const int per = (groups + cap - 1) / cap;
  int blocks = (groups + per - 1) / per;
  if (blocks >= kXcds * 4) blocks = (blocks + kXcds - 1) / kXcds * kXcds;
  return blocks;
}

template <int R, int U, int EPI>
void launch(const GemvParams& p, hipStream_t s, int cap) {
  const bool lds = p.K <= kMaxLdsK;
  const int groups = (p.N + kWaves * R - 1) / (kWaves * R);
  const int blocks = balanced_blocks(groups, cap);
  const size_t shm = lds ? (size_t)p.K * sizeof(float) : 0;
  if (p.norm_w) {
    if (!lds) ST_DIE("GEMV with RMSNorm needs K <= 16384");
    hipLaunchKernelGGL((gemv_kernel<R, U, EPI, true, true>), dim3(blocks), dim3(kThreads), shm, s, p);
  } else if (lds) {
    hipLaunchKernelGGL((gemv_kernel<R, U, EPI, false, true>), dim3(blocks), dim3(kThreads), shm, s, p);
  } else {
    hipLaunchKernelGGL((gemv_kernel<R, U, EPI, false, false>), dim3(blocks), dim3(kThreads), 0, s, p);
  }
}

void check(const GemvParams& p, int epi) {
  if (p.K <= 0 || p.K % 8 != 0) ST_DIE("GEMV needs K to be a positive multiple of 8");
  if (p.N <= 0) ST_DIE("GEMV needs N > 0");
  if (((uintptr_t)p.w | (uintptr_t)p.x) % 16 != 0) ST_DIE("GEMV operands must be 16-byte aligned");
  if (epi == GEMV_SWIGLU && (!p.w2 || (uintptr_t)p.w2 % 16)) ST_DIE("GEMV SwiGLU needs an aligned up matrix");
  if (epi == GEMV_QKV && p.N != p.q_dim + 2 * p.kv_dim) ST_DIE("GEMV QKV row count mismatch");
}

}  // namespace

void gemv(const GemvParams& p, int epi, hipStream_t s) {
  check(p, epi);
  switch (epi) {
    case GEMV_STORE: launch<1, 2, GEMV_STORE>(p, s, 2048); break;
    case GEMV_RESIDUAL: launch<1, 4, GEMV_RESIDUAL>(p, s, 4096); break;
    case GEMV_QKV: launch<1, 2, GEMV_QKV>(p, s, 2048); break;
    case GEMV_SWIGLU: launch<1, 2, GEMV_SWIGLU>(p, s, 2048); break;
    default: ST_DIE("unknown GEMV epilogue");
  }
  HIP_CHECK(hipGetLastError());
}

// Launch-shape variants for the micro-benchmark (STORE epilogue, or
// SwiGLU when `dual`): rows per wavefront R, steps per chunk U, block cap.
int gemv_variant_count() { return 12; }

void gemv_variant(const GemvParams& p, bool dual, int v, hipStream_t s) {
  check(p, dual ? GEMV_SWIGLU : GEMV_STORE);
#define V(R, U, CAP)                                                   \
  if (dual) launch<R, U, GEMV_SWIGLU>(p, s, CAP);                      \
  else launch<R, U, GEMV_STORE>(p, s, CAP);                            \
  break;
  switch (v) {
    case 0: V(1, 2, 2048)
    case 1: V(1, 4, 2048)
    case 2: V(1, 8, 2048)
    case 3: V(2, 2, 2048)
    case 4: V(2, 4, 2048)
    case 5: V(4, 2, 2048)
    case 6: V(1, 4, 1024)
    case 7: V(2, 4, 1024)
    case 8: V(1, 4, 512)
    case 9: V(2, 2, 512)
    case 10: V(4, 4, 1024)
    case 11: V(1, 4, 4096)
    default: ST_DIE("unknown GEMV variant");
  }
#undef V
  HIP_CHECK(hipGetLastError());
}

}  // namespace sg
