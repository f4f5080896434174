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

  const int P = EPI == GEMV_QKV ? *p.pos : 0;  // (before any store: as gemv_store)
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
            const size_t at = ((size_t)head * p.ctx + P) * p.head_dim + h;
            if (p.kv_bf16) ((uint16_t*)p.vcache)[at] = f32_to_bf16_any(acc[r]);
            else p.vcache[at] = acc[r];
          }
        }
      }
    }
  }
}

// Second form: one row per wavefront at a time and a flat stream of
// (row, step) items per wavefront, PD steps in flight in a ring of
// registers whose slots are fixed by unrolling (no register copies, so no
// wait is forced before a slot is consumed), running across row
// boundaries. The input row (and the RMSNorm weights) are loaded into
// registers before any weight load, so staging them waits for those loads
// alone while the first PD weight loads are in flight; the RMSNorm sum of
// squares is formed from the registers in the same partition and order as
// stage_row. Per row the products are accumulated in step order as in
// gemv_kernel; the row sum is a DPP reduction. Used when the staged row fits
// kV2Lds bytes and XF float4 per thread.
constexpr int kV2Lds = 64 * 1024;

// P: the step's position (*p.pos), read by the kernel before its first
// store: a read of it here, after the kernel's stores, would be a vector
// load that waits for every weight load in flight.
template <int EPI>
__device__ __forceinline__ void gemv_store(const GemvParams& p, int n, float a, float a2, int P) {
  if (EPI == GEMV_STORE) {
    p.y[n] = a;
  } else if (EPI == GEMV_RESIDUAL) {
    p.y[n] += a;
  } else if (EPI == GEMV_SWIGLU) {
    p.y[n] = silu_mul(a, a2);
  } else {  // GEMV_QKV
    if (n < p.q_dim) {
      p.q[n] = a;
    } else if (n < p.q_dim + p.kv_dim) {
      p.kraw[n - p.q_dim] = a;
    } else {
      const int j = n - p.q_dim - p.kv_dim;
      const int head = j / p.head_dim, h = j % p.head_dim;
      const size_t at = ((size_t)head * p.ctx + P) * p.head_dim + h;
      if (p.kv_bf16) ((uint16_t*)p.vcache)[at] = f32_to_bf16_any(a);
      else p.vcache[at] = a;
    }
  }
}

// The residual epilogue's y values of a wavefront's rows r < WAVE (row
// (g0 + r) * wv + wave in lane r), loaded before the weight stream. Read at
// a row's end instead, each would wait for every weight load in flight (a
// load completes in issue order), draining the ring once per row: with the
// input row in registers and an 8-deep ring (Llama-3.2-1B O and down) that
// cost 2.9% of the decode step; the LDS-staged third form, with more
// wavefronts per SIMD to cover the drain, measured no better with it.
template <int EPI>
__device__ __forceinline__ float residual_ahead(const GemvParams& p, int g0, int wv, int wave, int nrows,
                                                int lane) {
  return EPI == GEMV_RESIDUAL && lane < nrows ? p.y[(size_t)(g0 + lane) * wv + wave] : 0.0f;
}

// Row n's result a (and a2): the residual epilogue adds y[n] as held in
// lane rowi of yr by residual_ahead (rows past the first WAVE read it).
template <int EPI>
__device__ __forceinline__ void gemv_store_row(const GemvParams& p, int n, int rowi, float yr, float a, float a2,
                                               int lane, int P) {
  if (EPI == GEMV_RESIDUAL && rowi < WAVE) {
    const float y = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(yr), rowi));
    if (lane == 0) p.y[n] = y + a;
  } else if (lane == 0) {
    gemv_store<EPI>(p, n, a, a2, P);
  }
}

template <int EPI, bool NORM, int XF, bool EXACT, int kPD>
__global__ __launch_bounds__(kThreads) void gemv2_kernel(GemvParams p) {
  extern __shared__ __attribute__((aligned(16))) float xs[];  // [S * kStep], zero past K
  __shared__ float red[kWaves];
  constexpr bool DUAL = EPI == GEMV_SWIGLU;
  const int lane = threadIdx.x % WAVE;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);  // wave-uniform from here
  const int K = p.K, N = p.N;
  const int S = (K + kStep - 1) / kStep;  // steps per row
  const int groups = (N + kWaves - 1) / kWaves;
  const int G = gridDim.x, per = (groups + G - 1) / G;
  const int v = (G % kXcds == 0) ? (blockIdx.x % kXcds) * (G / kXcds) + blockIdx.x / kXcds : blockIdx.x;
  const int g0 = v * per;
  // rows of this wavefront: (g0 + i) * 4 + wave, i < nrows
  const int glast = N - 1 - wave >= 0 ? (N - 1 - wave) / kWaves : -1;  // last group with a row here
  const int nrows = max(0, min(min(groups, g0 + per), glast + 1) - g0);
  const int T = nrows * S;

  // input row elements tid*4 + i*1024 (and their norm weights), clamped
  float4 xv[XF];
  uint2 nv[NORM ? XF : 1];
#pragma unroll
  for (int i = 0; i < XF; i++) {
    const int k = min((int)threadIdx.x * 4 + i * kThreads * 4, K - 4);
    xv[i] = *(const float4*)(p.x + k);
    if (NORM) nv[i] = *(const uint2*)(p.norm_w + k);
  }
  const float yr = residual_ahead<EPI>(p, g0, kWaves, wave, nrows, lane);
  const int P = EPI == GEMV_QKV ? *p.pos : 0;

  // The ring. The refill cursor (rrow, rstep) walks the items in order.
  // Refills past the last item are issued all the same (so that every
  // consumption waits for an exact count of newer loads) but read the
  // first 1 KiB of the input row, which is in cache, instead of weights;
  // the up matrix's refills there read the neighbouring lane's 16 bytes
  // (at the gate refill's own address the compiler reuses that load's
  // value, a copy that waits for every load in flight at each refill).
  uint4 w[kPD], w2[DUAL ? kPD : 1];
  const int lk = lane * 8;
  int rrow = 0, rstep = 0;
  auto load = [&](uint4& a, uint4& b) {
    const bool past = rrow >= nrows;  // wave-uniform
    const size_t row = (size_t)min((g0 + rrow) * kWaves + wave, N - 1);
    const int k = EXACT ? rstep * kStep + lk : min(rstep * kStep + lk, K - 8);
    const uint16_t* wa = past ? (const uint16_t*)p.x + lk : p.w + row * K + k;
    a = load_nt_u4(wa);
    if (DUAL) b = load_nt_u4(past ? (const uint16_t*)p.x + (lk ^ 8) : p.w2 + row * K + k);
    if (++rstep == S) {
      rstep = 0;
      rrow++;
    }
  };
#pragma unroll
  for (int j = 0; j < kPD; j++) load(w[j], w2[DUAL ? j : 0]);
  __builtin_amdgcn_sched_barrier(0);  // the weight loads go out before the staging waits

  float s = 1.0f;
  if (NORM) {  // same partition and order as stage_row
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < XF; i++) {
      if ((int)threadIdx.x * 4 + i * kThreads * 4 < K) {
        ss = fmaf(xv[i].x, xv[i].x, ss);
        ss = fmaf(xv[i].y, xv[i].y, ss);
        ss = fmaf(xv[i].z, xv[i].z, ss);
        ss = fmaf(xv[i].w, xv[i].w, ss);
      }
    }
    s = rms_scale(block_sum<kThreads>(ss, red), K, p.eps);
  }
#pragma unroll
  for (int i = 0; i < XF; i++) {
    const int k = (int)threadIdx.x * 4 + i * kThreads * 4;
    if (k < K) {
      float4 o = xv[i];
      if (NORM) {
        o.x = (o.x * s) * bf16_to_f32((uint16_t)(nv[i].x & 0xffffu));
        o.y = (o.y * s) * bf16_to_f32((uint16_t)(nv[i].x >> 16));
        o.z = (o.z * s) * bf16_to_f32((uint16_t)(nv[i].y & 0xffffu));
        o.w = (o.w * s) * bf16_to_f32((uint16_t)(nv[i].y >> 16));
      }
      *(float4*)(xs + k) = o;
    }
  }
  for (int k = K + threadIdx.x; k < S * kStep; k += kThreads) xs[k] = 0.0f;
  __syncthreads();

  float acc = 0.0f, acc2 = 0.0f;
  int step = 0, rowi = 0;
  for (int t0 = 0; t0 < T; t0 += kPD) {
#pragma unroll
    for (int j = 0; j < kPD; j++) {
      if (t0 + j < T) {
        const int k = step * kStep + lk;
        uint4 a = w[j], b = w2[DUAL ? j : 0];
        if (!EXACT) {  // past K: zero weights (x is zero there too)
          const bool in = k < K;
          a.x = in ? a.x : 0u;
          a.y = in ? a.y : 0u;
          a.z = in ? a.z : 0u;
          a.w = in ? a.w : 0u;
          b.x = in ? b.x : 0u;
          b.y = in ? b.y : 0u;
          b.z = in ? b.z : 0u;
          b.w = in ? b.w : 0u;
        }
        const float4 xa = *(const float4*)(xs + k);
        const float4 xb = *(const float4*)(xs + k + 4);
        acc = dot8(a, xa, xb, acc);
        if (DUAL) acc2 = dot8(b, xa, xb, acc2);
        if (++step == S) {
          const float r1 = wave_total(acc), r2 = DUAL ? wave_total(acc2) : 0.0f;
          gemv_store_row<EPI>(p, (g0 + rowi) * kWaves + wave, rowi, yr, r1, r2, lane, P);
          acc = acc2 = 0.0f;
          step = 0;
          rowi++;
        }
      }
      load(w[j], w2[DUAL ? j : 0]);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);  // no load left in flight at exit
}

// Third form: gemv2's flat stream, with the input row staged by the
// global-to-LDS DMA instead of through registers. Order of issue: the
// RMSNorm weights of this thread (registers, K / 1024 uint2 at most
// kV3Nw), the DMA of the row (no registers held), then the first PD weight
// loads of the ring; waiting until only the ring loads are in flight
// completes the first two. The RMSNorm is then applied in LDS. Without the
// row in registers a wavefront holds the ring and little else, so more
// wavefronts (and weight bytes) are in flight per CU.
constexpr int kV3Nw = 8;  // uint2 of norm weights per thread: K <= 8192 with RMSNorm

typedef __attribute__((address_space(3))) void* lds_ptr_t;


// Waits until at most N vector-memory operations of this wavefront are in
// flight (N <= 63).
template <int N>
__device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_sched_barrier(0);
  // s_waitcnt encoding (gfx9): vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] << 14
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Sum over y < ny (at most YMAX) of part[y * stride], in y order, with
// every partial requested (agent-coherently) before the first is added.
template <int YMAX>
__device__ __forceinline__ float sum_parts(const float* part, size_t stride, int ny) {
  float v[YMAX];
#pragma unroll
  for (int y = 0; y < YMAX; y++) v[y] = y < ny ? cload(part + (size_t)y * stride) : 0.0f;
  float sum = v[0];
#pragma unroll
  for (int y = 1; y < YMAX; y++)
    if (y < ny) sum += v[y];
  return sum;
}
constexpr int kSplitRangesMax = 8;   // K ranges of the split-K third form
constexpr int kRowsRangesMax = 16;   // K ranges of the split-K rows form

// SPLIT (residual epilogue, no RMSNorm): block (x, y) takes the rows of x
// over K range y of gridDim.y ranges of whole steps: its row sums are
// partial sums, stored agent-coherently to p.part[y][n]; the last of the
// gridDim.y blocks of a row range to arrive (counter p.counters[x]) adds
// them in range order, y[n] += (part[0][n] + part[1][n]) + ..., and resets
// the counter. Rows longer than an LDS stage (64 KiB of fp32) take this
// path: each block stages only its range.
template <int EPI, bool NORM, bool EXACT, int kPD, bool SPLIT = false>
__global__ __launch_bounds__(kThreads) void gemv3_kernel(GemvParams p) {
  constexpr int NT = kThreads, WV = kWaves;
  extern __shared__ __attribute__((aligned(16))) float xs[];  // [S * kStep], zero past K
  __shared__ float red[WV];
  __shared__ int last;
  constexpr bool DUAL = EPI == GEMV_SWIGLU;
  static_assert(!SPLIT || (EPI == GEMV_RESIDUAL && !NORM), "split-K rows: residual epilogue only");
  constexpr int LOADS = kPD * (DUAL ? 2 : 1);  // ring loads issued before the staging wait
  const int lane = threadIdx.x % WAVE;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
  const int N = p.N, KR = p.K;  // KR: row length (stride of the weight rows)
  const int SR = (KR + kStep - 1) / kStep, SP = SPLIT ? (SR + gridDim.y - 1) / gridDim.y : SR;
  const int kbeg = SPLIT ? blockIdx.y * SP * kStep : 0;
  const int K = SPLIT ? min(KR - kbeg, SP * kStep) : KR;  // this block's K range
  const float* x = p.x + kbeg;
  const uint16_t* wbase = p.w + kbeg;
  const int S = (K + kStep - 1) / kStep;
  const int groups = (N + WV - 1) / WV;
  const int G = gridDim.x, per = (groups + G - 1) / G;
  const int v = (G % kXcds == 0) ? (blockIdx.x % kXcds) * (G / kXcds) + blockIdx.x / kXcds : blockIdx.x;
  const int g0 = v * per;
  const int glast = N - 1 - wave >= 0 ? (N - 1 - wave) / WV : -1;
  const int nrows = max(0, min(min(groups, g0 + per), glast + 1) - g0);
  const int T = nrows * S;

  // 1. this thread's RMSNorm weights (elements tid*4 + i*1024), the position
  const int P = EPI == GEMV_QKV ? *p.pos : 0;
  uint2 nv[NORM ? kV3Nw : 1];
  if (NORM) {
#pragma unroll
    for (int i = 0; i < kV3Nw; i++) {
      const int k = min((int)threadIdx.x * 4 + i * NT * 4, K - 4);
      nv[i] = *(const uint2*)(p.norm_w + k);
    }
  }
  // 2. the row into LDS: 16 bytes per lane, 1 KiB per wavefront instruction
  const int slots = K / 4;
  for (int u0 = wave * WAVE; u0 < slots; u0 += NT) {
    const int u = u0 + lane;
    if (u < slots)  // inactive lanes write nothing
      dma16_hidden(x + u * 4, (lds_ptr_t)(xs + u0 * 4));
  }
  __builtin_amdgcn_sched_barrier(0);  // the row's DMA is issued before the ring loads
  // 3. the ring
  uint4 w[kPD], w2[DUAL ? kPD : 1];
  const int lk = lane * 8;
  int rrow = 0, rstep = 0;
  auto load = [&](uint4& a, uint4& b) {
    const bool past = rrow >= nrows;  // wave-uniform
    const size_t row = (size_t)min((g0 + rrow) * WV + wave, N - 1);
    const int k = EXACT ? rstep * kStep + lk : min(rstep * kStep + lk, K - 8);
    const uint16_t* wa = past ? (const uint16_t*)p.x + lk : wbase + row * KR + k;
    a = load_nt_u4(wa);
    if (DUAL) b = load_nt_u4(past ? (const uint16_t*)p.x + (lk ^ 8) : p.w2 + row * KR + k);  // (as gemv2)
    if (++rstep == S) {
      rstep = 0;
      rrow++;
    }
  };
#pragma unroll
  for (int j = 0; j < kPD; j++) load(w[j], w2[DUAL ? j : 0]);
  wait_vm<LOADS>();  // norm weights and row landed; the ring stays in flight
  __syncthreads();
  for (int k = K + threadIdx.x; k < S * kStep; k += NT) xs[k] = 0.0f;
  if (NORM) {  // (x * s) * w in LDS, the sum of squares in stage_row's partition and order
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < kV3Nw; i++) {
      const int k = (int)threadIdx.x * 4 + i * NT * 4;
      if (k < K) {
        const float4 xv = *(const float4*)(xs + k);
        ss = fmaf(xv.x, xv.x, ss);
        ss = fmaf(xv.y, xv.y, ss);
        ss = fmaf(xv.z, xv.z, ss);
        ss = fmaf(xv.w, xv.w, ss);
      }
    }
    const float sc = rms_scale(block_sum<NT>(ss, red), K, p.eps);  // (contains a barrier)
#pragma unroll
    for (int i = 0; i < kV3Nw; i++) {
      const int k = (int)threadIdx.x * 4 + i * NT * 4;
      if (k < K) {
        float4 o = *(const float4*)(xs + k);
        o.x = (o.x * sc) * bf16_to_f32((uint16_t)(nv[i].x & 0xffffu));
        o.y = (o.y * sc) * bf16_to_f32((uint16_t)(nv[i].x >> 16));
        o.z = (o.z * sc) * bf16_to_f32((uint16_t)(nv[i].y & 0xffffu));
        o.w = (o.w * sc) * bf16_to_f32((uint16_t)(nv[i].y >> 16));
        *(float4*)(xs + k) = o;
      }
    }
  }
  __syncthreads();

  float acc = 0.0f, acc2 = 0.0f;
  int step = 0, rowi = 0;
  for (int t0 = 0; t0 < T; t0 += kPD) {
#pragma unroll
    for (int j = 0; j < kPD; j++) {
      if (t0 + j < T) {
        const int k = step * kStep + lk;
        uint4 a = w[j], b = w2[DUAL ? j : 0];
        if (!EXACT) {  // past K: zero weights (x is zero there too)
          const bool in = k < K;
          a.x = in ? a.x : 0u;
          a.y = in ? a.y : 0u;
          a.z = in ? a.z : 0u;
          a.w = in ? a.w : 0u;
          b.x = in ? b.x : 0u;
          b.y = in ? b.y : 0u;
          b.z = in ? b.z : 0u;
          b.w = in ? b.w : 0u;
        }
        const float4 xa = *(const float4*)(xs + k);
        const float4 xb = *(const float4*)(xs + k + 4);
        acc = dot8(a, xa, xb, acc);
        if (DUAL) acc2 = dot8(b, xa, xb, acc2);
        if (++step == S) {
          const float r1 = wave_total(acc), r2 = DUAL ? wave_total(acc2) : 0.0f;
          const int n = (g0 + rowi) * WV + wave;
          if (lane == 0) {
            if (SPLIT) cstore(p.part + (size_t)blockIdx.y * N + n, r1);
            else gemv_store<EPI>(p, n, r1, r2, P);
          }
          acc = acc2 = 0.0f;
          step = 0;
          rowi++;
        }
      }
      load(w[j], w2[DUAL ? j : 0]);
    }
  }
  compiler_fence();
  __builtin_amdgcn_s_waitcnt(0);  // no load left in flight, every partial stored
  if (!SPLIT) return;
  // Hand-off (the decode attention's): partials are written and read only
  // by agent-scope relaxed atomic accesses, every store of the block has
  // completed before the counter increment is issued, and the last block
  // reads after its own increment has returned.
  __syncthreads();
  if (threadIdx.x == 0) {
    const unsigned done = __hip_atomic_fetch_add(p.counters + blockIdx.x, 1u, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
    last = done == gridDim.y - 1;
  }
  __syncthreads();
  if (!last) return;
  compiler_fence();
  const int n_end = min(N, min(groups, g0 + per) * WV);
  for (int n = g0 * WV + (int)threadIdx.x; n < n_end; n += NT) {
    p.y[n] += sum_parts<kSplitRangesMax>(p.part + n, N, gridDim.y);
  }
  if (threadIdx.x == 0) __hip_atomic_store(p.counters + blockIdx.x, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ------------------------------------------------------------ rows form --
// The third form for M <= MM activation rows (prefill of a few tokens): the
// block stages the M rows of its K range in LDS ([MM][S * kStep] fp32, zero
// past K and past row M; the RMSNorm of each row when NORM), and each
// wavefront streams one weight row at a time through the fixed-slot
// register ring of gemv3, multiplying every 512-element step with all MM
// rows: per activation row and lane the decode GEMV's fp32 FMAs in step
// order, so each weight row is read from HBM once for all rows. The MM row
// sums of a weight row are reduced together (multi_total).

// Sum over the 64 lanes of each of MM (1, 2, 4 or 8) per-lane values: in
// rounds over lane bits 5, 4, ... each lane keeps half of its values (the
// upper half where the bit is set) and adds its partner's copy of them, so
// after log2(MM) rounds a lane holds one value, that of row
// lane >> (6 - log2(MM)), summed over the lanes that differ in those bits;
// the remaining rounds sum over the other lane bits.
template <int MM, int BIT = 32>
__device__ __forceinline__ float multi_total(const float (&a)[MM], int lane) {
  if constexpr (MM == 1) {
    float v = a[0];
#pragma unroll
    for (int b = BIT; b >= 1; b >>= 1) v += __shfl_xor(v, b, WAVE);
    return v;
  } else {
    constexpr int H = MM / 2;
    const bool up = (lane & BIT) != 0;
    float h[H];
#pragma unroll
    for (int i = 0; i < H; i++) {
      const float send = up ? a[i] : a[i + H];
      const float keep = up ? a[i + H] : a[i];
      h[i] = keep + __shfl_xor(send, BIT, WAVE);
    }
    return multi_total<H, BIT / 2>(h, lane);
  }
}

// The eight bf16 weights of a 16-byte load as fp32 (exact), and their dot
// product with eight fp32 values in element order (dot8's arithmetic).
__device__ __forceinline__ void widen8(uint4 w, float (&f)[8]) {
  f[0] = bf16_lo(w.x);
  f[1] = bf16_hi(w.x);
  f[2] = bf16_lo(w.y);
  f[3] = bf16_hi(w.y);
  f[4] = bf16_lo(w.z);
  f[5] = bf16_hi(w.z);
  f[6] = bf16_lo(w.w);
  f[7] = bf16_hi(w.w);
}
__device__ __forceinline__ float dot8f(const float (&f)[8], const float4& a, const float4& b, float acc) {
  acc = fmaf(f[0], a.x, acc);
  acc = fmaf(f[1], a.y, acc);
  acc = fmaf(f[2], a.z, acc);
  acc = fmaf(f[3], a.w, acc);
  acc = fmaf(f[4], b.x, acc);
  acc = fmaf(f[5], b.y, acc);
  acc = fmaf(f[6], b.z, acc);
  acc = fmaf(f[7], b.w, acc);
  return acc;
}

template <int MM>
constexpr int log2_rows() {
  return MM == 1 ? 0 : MM == 2 ? 1 : MM == 4 ? 2 : 3;
}

template <int EPI, int MM, bool SPLIT>
__device__ __forceinline__ void gemvm_store(const GemvParams& p, int m, int n, float a, float a2, int P) {
  const int N = p.N;
  if (SPLIT) {
    cstore(p.part + ((size_t)blockIdx.y * MM + m) * N + n, a);
  } else if (EPI == GEMV_STORE) {
    p.y[(size_t)m * N + n] = a;
  } else if (EPI == GEMV_RESIDUAL) {
    p.y[(size_t)m * N + n] += a;
  } else if (EPI == GEMV_SWIGLU) {
    p.y[(size_t)m * N + n] = silu_mul(a, a2);
  } else {  // GEMV_QKV: q, keys (cache or staging), values at position P + m
    if (n < p.q_dim) {
      p.q[(size_t)m * p.q_dim + n] = a;
    } else if (n < p.q_dim + p.kv_dim) {
      const int j = n - p.q_dim;
      if (p.kv_bf16) {
        p.kstage[(size_t)m * p.kv_dim + j] = a;  // rounded after its RoPE
      } else {
        const int head = j / p.head_dim, h = j % p.head_dim;
        p.kcache[((size_t)head * p.ctx + P + m) * p.head_dim + h] = a;
      }
    } else {
      const int j = n - p.q_dim - p.kv_dim;
      const int head = j / p.head_dim, h = j % p.head_dim;
      const size_t at = ((size_t)head * p.ctx + P + m) * p.head_dim + h;
      if (p.kv_bf16) ((uint16_t*)p.vcache)[at] = f32_to_bf16_any(a);
      else p.vcache[at] = a;
    }
  }
}

// SPLIT (residual epilogue, no RMSNorm): block (x, y) takes the rows of x
// over K range y; row sums go to p.part[y][m][n] (agent-coherent) and the
// last block of a row range to arrive adds them in range order, as in
// gemv3_kernel's split form.
constexpr int kRowsThreads = 512;  // eight wavefronts share one staging of the rows

// R weight rows per wavefront at a time: every activation value read from
// LDS serves R rows (LDS traffic per weight byte / R); the launcher lowers
// R where R rows per wavefront would leave CUs without a block.
template <int MM, int EPI, bool NORM, bool EXACT, int kPD, bool SPLIT, int R>
__global__ __launch_bounds__(kRowsThreads) void gemvm_kernel(GemvParams p) {
  constexpr int NT = kRowsThreads, WV = NT / WAVE;
  extern __shared__ __attribute__((aligned(16))) float xs[];  // [MM][S * kStep]
  __shared__ float red[MM][WV];
  __shared__ int last;
  constexpr bool DUAL = EPI == GEMV_SWIGLU;
  static_assert(!SPLIT || (EPI == GEMV_RESIDUAL && !NORM), "split-K rows: residual epilogue only");
  constexpr int LOADS = kPD * R * (DUAL ? 2 : 1);  // ring loads issued before the staging wait
  const int lane = threadIdx.x % WAVE;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
  const int N = p.N, KR = p.K, M = p.M;
  const int SR = (KR + kStep - 1) / kStep, SP = SPLIT ? (SR + gridDim.y - 1) / gridDim.y : SR;
  const int kbeg = SPLIT ? blockIdx.y * SP * kStep : 0;
  const int K = SPLIT ? min(KR - kbeg, SP * kStep) : KR;  // this block's K range
  const int S = (K + kStep - 1) / kStep, LD = S * kStep;
  const uint16_t* wbase = p.w + kbeg;
  // a group is WV * R rows: wavefront w takes rows (group * WV + w) * R + r
  const int groups = (N + WV * R - 1) / (WV * R);
  const int G = gridDim.x, per = (groups + G - 1) / G;
  const int v = (G % kXcds == 0) ? (blockIdx.x % kXcds) * (G / kXcds) + blockIdx.x / kXcds : blockIdx.x;
  const int g0 = v * per;
  const int glast = N - 1 - wave * R >= 0 ? (N - 1 - wave * R) / (WV * R) : -1;
  const int nrows = max(0, min(min(groups, g0 + per), glast + 1) - g0);  // row sets of R
  const int T = nrows * S;

  // 1. this thread's RMSNorm weights (elements tid*4 + i*NT*4), the
  // position (read here, before any store: as gemv_store)
  const int P = EPI == GEMV_QKV ? *p.pos : 0;
  uint2 nv[NORM ? kV3Nw : 1];
  if (NORM) {
#pragma unroll
    for (int i = 0; i < kV3Nw; i++) {
      const int k = min((int)threadIdx.x * 4 + i * NT * 4, K - 4);
      nv[i] = *(const uint2*)(p.norm_w + k);
    }
  }
  // 2. the M rows into LDS: 16 bytes per lane, 1 KiB per wavefront instruction
  const int slots = K / 4;
  for (int m = 0; m < M; m++) {
    const float* xr = p.x + (size_t)m * KR + kbeg;
    float* dst = xs + m * LD;
    for (int u0 = wave * WAVE; u0 < slots; u0 += NT) {
      const int u = u0 + lane;
      if (u < slots)  // inactive lanes write nothing
        dma16_hidden(xr + u * 4, (lds_ptr_t)(dst + u0 * 4));
    }
  }
  __builtin_amdgcn_sched_barrier(0);  // the rows' DMA is issued before the ring loads
  // 3. the ring: kPD steps of R rows (and their up rows)
  uint4 w[kPD][R], w2[DUAL ? kPD : 1][R];
  const int lk = lane * 8;
  int rrow = 0, rstep = 0;
  auto load = [&](uint4 (&a)[R], uint4 (&b)[R]) {
    // past this wave's rows: loads inside row N - 1 (never multiplied)
    const bool past = rrow >= nrows;  // wave-uniform
    const int k = past ? min(lk, K - 8) : EXACT ? rstep * kStep + lk : min(rstep * kStep + lk, K - 8);
#pragma unroll
    for (int r = 0; r < R; r++) {
      const size_t row = past ? (size_t)(N - 1) : (size_t)min(((g0 + rrow) * WV + wave) * R + r, N - 1);
      a[r] = load_nt_u4(wbase + row * KR + k);
      if (DUAL) b[r] = load_nt_u4(p.w2 + kbeg + row * KR + k);
    }
    if (++rstep == S) {
      rstep = 0;
      rrow++;
    }
  };
#pragma unroll
  for (int j = 0; j < kPD; j++) load(w[j], w2[DUAL ? j : 0]);
  wait_vm<LOADS>();  // norm weights and rows landed; the ring stays in flight
  __syncthreads();
  for (int m = 0; m < MM; m++)  // zero past K, and rows past M
    for (int k = (m < M ? K : 0) + threadIdx.x; k < LD; k += NT) xs[m * LD + k] = 0.0f;
  if (NORM) {  // (x * s) * w per row
    float ss[MM];
#pragma unroll
    for (int m = 0; m < MM; m++) ss[m] = 0.0f;
#pragma unroll
    for (int i = 0; i < kV3Nw; i++) {
      const int k = (int)threadIdx.x * 4 + i * NT * 4;
      if (k < K) {
#pragma unroll
        for (int m = 0; m < MM; m++) {  // rows past M are zero
          const float4 xv = *(const float4*)(xs + m * LD + k);
          ss[m] = fmaf(xv.x, xv.x, ss[m]);
          ss[m] = fmaf(xv.y, xv.y, ss[m]);
          ss[m] = fmaf(xv.z, xv.z, ss[m]);
          ss[m] = fmaf(xv.w, xv.w, ss[m]);
        }
      }
    }
#pragma unroll
    for (int m = 0; m < MM; m++) {
      const float t = wave_total(ss[m]);
      if (lane == 0) red[m][wave] = t;
    }
    __syncthreads();
    float sc[MM];
#pragma unroll
    for (int m = 0; m < MM; m++) {
      float t = 0.0f;
#pragma unroll
      for (int i = 0; i < WV; i++) t += red[m][i];
      sc[m] = rms_scale(t, K, p.eps);
    }
#pragma unroll
    for (int i = 0; i < kV3Nw; i++) {
      const int k = (int)threadIdx.x * 4 + i * NT * 4;
      if (k < K) {
        const float n0 = bf16_to_f32((uint16_t)(nv[i].x & 0xffffu)), n1 = bf16_to_f32((uint16_t)(nv[i].x >> 16));
        const float n2 = bf16_to_f32((uint16_t)(nv[i].y & 0xffffu)), n3 = bf16_to_f32((uint16_t)(nv[i].y >> 16));
#pragma unroll
        for (int m = 0; m < MM; m++) {
          float4 o = *(const float4*)(xs + m * LD + k);
          o.x = (o.x * sc[m]) * n0;
          o.y = (o.y * sc[m]) * n1;
          o.z = (o.z * sc[m]) * n2;
          o.w = (o.w * sc[m]) * n3;
          *(float4*)(xs + m * LD + k) = o;
        }
      }
    }
  }
  __syncthreads();

  float acc[R][MM], acc2[DUAL ? R : 1][MM];
#pragma unroll
  for (int r = 0; r < R; r++)
#pragma unroll
    for (int m = 0; m < MM; m++) acc[r][m] = acc2[DUAL ? r : 0][m] = 0.0f;
  const int mrow = lane >> (6 - log2_rows<MM>());  // the activation row this lane stores
  const bool storer = (lane & ((WAVE / MM) - 1)) == 0 && mrow < M;
  int step = 0, rowi = 0;
  for (int t0 = 0; t0 < T; t0 += kPD) {
#pragma unroll
    for (int j = 0; j < kPD; j++) {
      if (t0 + j < T) {
        const int k = step * kStep + lk;
        uint4 a[R], b[DUAL ? R : 1];
#pragma unroll
        for (int r = 0; r < R; r++) {
          a[r] = w[j][r];
          if (DUAL) b[r] = w2[DUAL ? j : 0][r];
        }
        if (!EXACT && k >= K) {  // past K: zero weights (the rows are zero there too)
#pragma unroll
          for (int r = 0; r < R; r++) {
            a[r] = make_uint4(0u, 0u, 0u, 0u);
            if (DUAL) b[r] = make_uint4(0u, 0u, 0u, 0u);
          }
        }
        // the weights widened once per step (exact), then MM rows of FMAs
        float wf[R][8], wg[DUAL ? R : 1][8];
#pragma unroll
        for (int r = 0; r < R; r++) {
          widen8(a[r], wf[r]);
          if (DUAL) widen8(b[DUAL ? r : 0], wg[DUAL ? r : 0]);
        }
#pragma unroll
        for (int m = 0; m < MM; m++) {
          const float4 xa = *(const float4*)(xs + m * LD + k);
          const float4 xb = *(const float4*)(xs + m * LD + k + 4);
#pragma unroll
          for (int r = 0; r < R; r++) {
            acc[r][m] = dot8f(wf[r], xa, xb, acc[r][m]);
            if (DUAL) acc2[DUAL ? r : 0][m] = dot8f(wg[DUAL ? r : 0], xa, xb, acc2[DUAL ? r : 0][m]);
          }
        }
        if (++step == S) {
#pragma unroll
          for (int r = 0; r < R; r++) {
            const float r1 = multi_total<MM>(acc[r], lane);
            float r2 = 0.0f;
            if constexpr (DUAL) r2 = multi_total<MM>(acc2[r], lane);
            const int n = ((g0 + rowi) * WV + wave) * R + r;
            if (storer && n < N) gemvm_store<EPI, MM, SPLIT>(p, mrow, n, r1, r2, P);
#pragma unroll
            for (int m = 0; m < MM; m++) acc[r][m] = acc2[DUAL ? r : 0][m] = 0.0f;
          }
          step = 0;
          rowi++;
        }
      }
      load(w[j], w2[DUAL ? j : 0]);
    }
  }
  compiler_fence();
  __builtin_amdgcn_s_waitcnt(0);  // no load left in flight, every partial stored
  if (!SPLIT) return;
  __syncthreads();  // (the hand-off of gemv3_kernel's split form)
  if (threadIdx.x == 0) {
    const unsigned done = __hip_atomic_fetch_add(p.counters + blockIdx.x, 1u, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
    last = done == gridDim.y - 1;
  }
  __syncthreads();
  if (!last) return;
  compiler_fence();
  const int n0 = g0 * WV * R, n_end = min(N, min(groups, g0 + per) * WV * R);
  for (int i = (int)threadIdx.x; i < (n_end - n0) * M; i += NT) {
    const int m = i / (n_end - n0), n = n0 + i % (n_end - n0);
    p.y[(size_t)m * N + n] += sum_parts<kRowsRangesMax>(p.part + (size_t)m * N + n, (size_t)MM * N, gridDim.y);
  }
  if (threadIdx.x == 0) __hip_atomic_store(p.counters + blockIdx.x, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Blocks: at most `cap`, the same number of row groups for each block, and
// a multiple of the XCD count when there are enough groups.
int balanced_blocks(int groups, int cap) {
  const int per = (groups + cap - 1) / cap;
  int blocks = (groups + per - 1) / per;
  if (blocks >= kXcds * 4) blocks = (blocks + kXcds - 1) / kXcds * kXcds;
  return blocks;
}

// PD: weight steps in flight per wavefront (8 KiB; the SwiGLU pair reads
// two matrices per step, so half as many steps).
template <int EPI, int PD = EPI == GEMV_SWIGLU ? 4 : 8>
bool launch_v2(const GemvParams& p, hipStream_t s, int cap) {
  const int S = (p.K + kStep - 1) / kStep;
  const size_t shm = (size_t)S * kStep * sizeof(float);
  if (shm > kV2Lds || p.K < 256 || p.K > 16 * kThreads * 4) return false;  // K >= 256: 1 KiB of x
  const int groups = (p.N + kWaves - 1) / kWaves;
  const int blocks = balanced_blocks(groups, cap);
  static bool attr = false;
  if (!attr) {
#define V2_ATTR(NORM, XF, EX)                                                                   \
  HIP_CHECK(hipFuncSetAttribute((const void*)gemv2_kernel<EPI, NORM, XF, EX, PD>,               \
                                hipFuncAttributeMaxDynamicSharedMemorySize, kV2Lds));
    V2_ATTR(true, 4, true)
    V2_ATTR(false, 4, true)
    V2_ATTR(true, 16, true)
    V2_ATTR(false, 16, true)
    V2_ATTR(true, 4, false)
    V2_ATTR(false, 4, false)
    V2_ATTR(true, 16, false)
    V2_ATTR(false, 16, false)
#undef V2_ATTR
    attr = true;
  }
  const bool small = p.K <= 4 * kThreads * 4, exact = p.K % kStep == 0;
#define V2_GO(NORM, XF, EX) \
  hipLaunchKernelGGL((gemv2_kernel<EPI, NORM, XF, EX, PD>), dim3(blocks), dim3(kThreads), shm, s, p)
#define V2_GO2(NORM, XF) \
  if (exact) V2_GO(NORM, XF, true); else V2_GO(NORM, XF, false);
  if (p.norm_w) {
    if (small) { V2_GO2(true, 4) }
    else { V2_GO2(true, 16) }
  } else {
    if (small) { V2_GO2(false, 4) }
    else { V2_GO2(false, 16) }
  }
#undef V2_GO2
#undef V2_GO
  return true;
}

// The third form; false when the row does not fit (K >= 256, up to 64 KiB
// of fp32 row; with RMSNorm K <= 8192).
template <int EPI, int PD>
bool launch_v3(const GemvParams& p, hipStream_t s, int cap) {
  const int S = (p.K + kStep - 1) / kStep;
  const size_t shm = (size_t)S * kStep * sizeof(float);
  if (shm > (size_t)kV2Lds || p.K < 256 || (p.norm_w && p.K > kV3Nw * kThreads * 4)) return false;
  const int groups = (p.N + kWaves - 1) / kWaves;
  const int blocks = balanced_blocks(groups, cap);
  static bool attr = false;
  if (!attr) {
    HIP_CHECK(hipFuncSetAttribute((const void*)gemv3_kernel<EPI, true, true, PD>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, kV2Lds));
    HIP_CHECK(hipFuncSetAttribute((const void*)gemv3_kernel<EPI, false, true, PD>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, kV2Lds));
    HIP_CHECK(hipFuncSetAttribute((const void*)gemv3_kernel<EPI, true, false, PD>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, kV2Lds));
    HIP_CHECK(hipFuncSetAttribute((const void*)gemv3_kernel<EPI, false, false, PD>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, kV2Lds));
    attr = true;
  }
  const bool exact = p.K % kStep == 0;
  if (p.norm_w) {
    if (exact) hipLaunchKernelGGL((gemv3_kernel<EPI, true, true, PD>), dim3(blocks), dim3(kThreads), shm, s, p);
    else hipLaunchKernelGGL((gemv3_kernel<EPI, true, false, PD>), dim3(blocks), dim3(kThreads), shm, s, p);
  } else {
    if (exact) hipLaunchKernelGGL((gemv3_kernel<EPI, false, true, PD>), dim3(blocks), dim3(kThreads), shm, s, p);
    else hipLaunchKernelGGL((gemv3_kernel<EPI, false, false, PD>), dim3(blocks), dim3(kThreads), shm, s, p);
  }
  return true;
}

// The split-K third form for rows longer than an LDS stage (residual
// epilogue without RMSNorm): ranges of at most kSplitSteps steps (32 KiB of
// fp32 row per block, so several blocks per CU), blockIdx.y = the range.
// Mistral-Small-24B down projection (K = 32768, 4 ranges): 57.5-58 us
// against 60.2 for the chunked form (row read from L2 per step); 128-768
// row blocks per range, 4-16 steps in flight and ranges of 8 or 32 steps
// measured the same.
constexpr int kSplitSteps = 16;
constexpr int kSplitMax = kSplitRangesMax;  // ranges: K <= 65536
template <int PD>
bool launch_v3_split(const GemvParams& p, hipStream_t s, int cap) {
  const int S = (p.K + kStep - 1) / kStep;
  const int ranges = (S + kSplitSteps - 1) / kSplitSteps;
  if (!p.part || !p.counters || p.norm_w || ranges < 2 || ranges > kSplitMax) return false;
  const int SP = (S + ranges - 1) / ranges;
  const size_t shm = (size_t)SP * kStep * sizeof(float);
  const int groups = (p.N + kWaves - 1) / kWaves;
  const int blocks = balanced_blocks(groups, cap);
  if (blocks > kGemvCounters) ST_DIE("GEMV split-K: more row ranges than counters");
  const bool exact = p.K % (SP * kStep) == 0;
  if (exact) hipLaunchKernelGGL((gemv3_kernel<GEMV_RESIDUAL, false, true, PD, true>), dim3(blocks, ranges),
                                dim3(kThreads), shm, s, p);
  else hipLaunchKernelGGL((gemv3_kernel<GEMV_RESIDUAL, false, false, PD, true>), dim3(blocks, ranges),
                          dim3(kThreads), shm, s, p);
  return true;
}

// The rows form: LDS for MM rows of the K range up to kRowsLds (one block
// of eight wavefronts per CU); rows with RMSNorm must fit whole, residual
// rows longer than that split over K (p.part / p.counters given).
constexpr int kRowsLds = 128 * 1024;
constexpr int kRowsSplitMax = kRowsRangesMax;

template <int MM, int EPI, bool NORM, bool EXACT, bool SPLIT, int R>
void rows_go_r(const GemvParams& p, dim3 grid, size_t shm, hipStream_t s) {
  constexpr int PD = R == 1 ? 4 : 2;  // steps of R rows in flight (R x 1 KiB each, twice for SwiGLU)
  static bool attr = false;
  if (!attr) {
    HIP_CHECK(hipFuncSetAttribute((const void*)gemvm_kernel<MM, EPI, NORM, EXACT, PD, SPLIT, R>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, kRowsLds));
    attr = true;
  }
  hipLaunchKernelGGL((gemvm_kernel<MM, EPI, NORM, EXACT, PD, SPLIT, R>), grid, dim3(kRowsThreads), shm, s, p);
}

// Rows per wavefront: the largest R (4, or 2 for the SwiGLU pair) whose
// groups of 8 R rows still give every CU a block (cap blocks in all).
inline int rows_r(int epi, int N, int cap_x) {
  const int rmax = epi == GEMV_SWIGLU ? 2 : 4;
  for (int r = rmax; r > 1; r /= 2)
    if ((N + 8 * r - 1) / (8 * r) >= cap_x) return r;
  return 1;
}

template <int MM, int EPI, bool NORM, bool EXACT, bool SPLIT>
void rows_go(const GemvParams& p, dim3 grid, size_t shm, int R, hipStream_t s) {
  if (R == 4 && EPI != GEMV_SWIGLU) rows_go_r<MM, EPI, NORM, EXACT, SPLIT, 4>(p, grid, shm, s);
  else if (R >= 2) rows_go_r<MM, EPI, NORM, EXACT, SPLIT, 2>(p, grid, shm, s);
  else rows_go_r<MM, EPI, NORM, EXACT, SPLIT, 1>(p, grid, shm, s);
}

template <int MM, int EPI>
bool launch_rows(const GemvParams& p, hipStream_t s, int cap) {
  const bool norm = p.norm_w != nullptr;
  const int S = (p.K + kStep - 1) / kStep;
  const int fit = kRowsLds / (MM * kStep * (int)sizeof(float));  // steps per LDS stage
  int ranges = (S + fit - 1) / fit;
  if (norm && (ranges > 1 || p.K > kV3Nw * kRowsThreads * 4)) return false;
  if (ranges > 1 && (EPI != GEMV_RESIDUAL || !p.part || !p.counters || ranges > kRowsSplitMax)) return false;
  const int SP = (S + ranges - 1) / ranges;
  ranges = (S + SP - 1) / SP;
  const size_t shm = (size_t)MM * SP * kStep * sizeof(float);
  const int cap_x = std::max(1, cap / ranges);  // cap blocks in all
  const int R = rows_r(EPI, p.N, cap_x);
  const int rows_per_group = kRowsThreads / WAVE * R;
  const int groups = (p.N + rows_per_group - 1) / rows_per_group;
  const int blocks = balanced_blocks(groups, cap_x);
  if (ranges > 1 && blocks > kGemvCounters) return false;
  const dim3 grid(blocks, ranges);
  const bool exact = p.K % kStep == 0;  // every range's steps then lie inside K
  if constexpr (EPI == GEMV_RESIDUAL) {
    if (ranges > 1) {
      if (exact) rows_go<MM, EPI, false, true, true>(p, grid, shm, R, s);
      else rows_go<MM, EPI, false, false, true>(p, grid, shm, R, s);
      return true;
    }
  }
  if (norm) {
    if (exact) rows_go<MM, EPI, true, true, false>(p, grid, shm, R, s);
    else rows_go<MM, EPI, true, false, false>(p, grid, shm, R, s);
  } else {
    if (exact) rows_go<MM, EPI, false, true, false>(p, grid, shm, R, s);
    else rows_go<MM, EPI, false, false, false>(p, grid, shm, R, s);
  }
  return true;
}

bool rows_fit(int M, int K, bool norm) {
  const int MM = M <= 4 ? 4 : 8;
  const int S = (K + kStep - 1) / kStep, fit = kRowsLds / (MM * kStep * (int)sizeof(float));
  const int ranges = (S + fit - 1) / fit;
  return M >= 1 && M <= kRowsMax && (norm ? ranges == 1 && K <= kV3Nw * kRowsThreads * 4 : ranges <= kRowsSplitMax);
}

template <int EPI>
bool rows_dispatch(const GemvParams& p, hipStream_t s) {
  constexpr int cap = 256;  // one block per CU: each CU stages the rows once (two per CU measured slower)
  if (p.M <= 4) return launch_rows<4, EPI>(p, s, cap);
  return launch_rows<8, EPI>(p, s, cap);
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

bool gemv_rows_fit(int M, int K, bool norm) { return rows_fit(M, K, norm); }

bool gemv_rows(const GemvParams& p, int epi, hipStream_t s) {
  check(p, epi);
  if (p.M < 1 || p.M > kRowsMax) ST_DIE("multi-row GEMV takes 1 to 8 activation rows");
  if (epi == GEMV_QKV && !p.kv_bf16 && !p.kcache) ST_DIE("multi-row QKV GEMV needs the key cache");
  if (epi == GEMV_QKV && p.kv_bf16 && !p.kstage) ST_DIE("multi-row QKV GEMV needs the key staging rows");
  bool ok = false;
  switch (epi) {
    case GEMV_STORE: ok = rows_dispatch<GEMV_STORE>(p, s); break;
    case GEMV_RESIDUAL: ok = rows_dispatch<GEMV_RESIDUAL>(p, s); break;
    case GEMV_QKV: ok = rows_dispatch<GEMV_QKV>(p, s); break;
    case GEMV_SWIGLU: ok = rows_dispatch<GEMV_SWIGLU>(p, s); break;
    default: ST_DIE("unknown GEMV epilogue");
  }
  if (ok) HIP_CHECK(hipGetLastError());
  return ok;
}

void gemv(const GemvParams& p, int epi, hipStream_t s) {
  check(p, epi);
  // Forms and launch shapes from sweeps of the decode shapes on MI355X
  // (weights streamed from HBM, back-to-back launches): the third form
  // (row staged by DMA) where it was faster, else the flat-stream form,
  // else, for rows beyond 64 KiB, the split-K third form (residual rows
  // given the scratch) or the chunked form.
  switch (epi) {
    case GEMV_STORE:  // logits
      if (!launch_v3<GEMV_STORE, 4>(p, s, 8192) && !launch_v2<GEMV_STORE, 8>(p, s, 2048))
        launch<1, 2, GEMV_STORE>(p, s, 2048);
      break;
    case GEMV_RESIDUAL:  // O and down projections
      if (!(p.N >= 2560 && launch_v3<GEMV_RESIDUAL, 4>(p, s, 768)) &&
          !launch_v2<GEMV_RESIDUAL, 8>(p, s, 256) && !launch_v3_split<8>(p, s, 256))
        launch<1, 4, GEMV_RESIDUAL>(p, s, 4096);
      break;
    case GEMV_QKV:  // the register-row form first up to K = 3072 (Llama-3.2-1B
      // 1563 -> 1578 tok/s, MXFP4 MoE 744 -> 751, Qwen3-4B 497 -> 498), the
      // third form above it (Mistral-Small-24B 127.7 -> 126.7 the other way)
      if (!(p.K <= 3072 && launch_v2<GEMV_QKV, 4>(p, s, 1024)) && !launch_v3<GEMV_QKV, 4>(p, s, 768) &&
          !launch_v2<GEMV_QKV, 4>(p, s, 1024))
        launch<1, 2, GEMV_QKV>(p, s, 2048);
      break;
    case GEMV_SWIGLU:  // gate/up: the third form pays from K > 4096, with 4
      // steps (8 loads) in flight: Mistral-Small-24B 106.1 -> 103.8 us
      // against 2 (3 the same; 768 or 2048 blocks slower)
      if (!(p.K > 4096 && launch_v3<GEMV_SWIGLU, 4>(p, s, 1024)) &&
          !launch_v2<GEMV_SWIGLU, 2>(p, s, 2048))
        launch<1, 2, GEMV_SWIGLU>(p, s, 2048);
      break;
    default: ST_DIE("unknown GEMV epilogue");
  }
  HIP_CHECK(hipGetLastError());
}

}  // namespace sg
