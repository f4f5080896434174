// Mixture-of-experts FFN kernels (no reference counterpart; semantics are
// defined by this library and restated by the CPU oracle):
//   router   logits_e = W_r[e] . xn (bf16 weights, fp32 accumulate),
//            the k largest in descending order (ties: lowest expert id),
//            weights = softmax over those k logits;
//   experts  a_j = silu(G_e xn) * (U_e xn) with MXFP4 G_e, U_e;
//            out = sum_j w_j (D_e a_j), accumulated in top-k order as
//            acc = fmaf(w_j, D_e a_j, acc), then x += acc.
// MXFP4 rows are [K/32] blocks of 16 code bytes (element 2i in the low
// nibble of byte i) and one E8M0 exponent each.
//
// Decode mapping: half a wavefront (32 lanes) per weight row, one 32-value
// block per lane per step (one 128-bit load plus its scale byte), every
// load of the wave's rows issued before the first is used; the block is
// decoded with v_cvt_scalef32_pk_f32_fp4 (E2M1 times the E8M0 scale, exact
// in fp32) and multiplied with the activation row staged in LDS.
//
// Algorithmic bytes per launch: the MXFP4 weights of the selected experts,
// K/2 + K/32 bytes per row.
#include "device_common.h"
#include "hip_check.h"
#include "kernels.h"

namespace sg {

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / WAVE;
constexpr int kHalves = 2 * kWaves;  // half-waves per block
constexpr int kSteps = 3;            // blocks of 32 values per lane per pass (96 per row)
constexpr int kGuRows = 2;           // rows per half-wave (gate/up)
constexpr int kDownRows = 1;         // rows per half-wave (down)

// Two values of byte `B` of `w` times `sc` (low nibble first).
template <int B>
__device__ __forceinline__ float2v fp4_pair(uint32_t w, float sc) {
  return __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, sc, B);
}

// A 32-value block (four code words) times `sc` as 16 packed bf16 pairs,
// element 2j in the low half of o[j]: one conversion per pair, exact (an
// E2M1 value times a power of two has at most two significant bits, inside
// bf16's exponent range, subnormals included).
typedef __bf16 bf16x2v_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ void fp4_block_bf16(const uint32_t (&w)[4], float sc, uint32_t (&o)[16]) {
#pragma unroll
  for (int i = 0; i < 4; i++) {
    o[4 * i + 0] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[i], sc, 0));
    o[4 * i + 1] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[i], sc, 1));
    o[4 * i + 2] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[i], sc, 2));
    o[4 * i + 3] = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(w[i], sc, 3));
  }
}

// Activation rows in LDS: rows of K values back to back, each 32-value
// block (8 chunks of 16 bytes) with chunk c stored at position c ^ (b & 7)
// of block b. Lanes that take consecutive blocks then read the same
// logical chunk from 8 different bank groups (without the swizzle every
// lane of a half-wave would hit the same four banks). The rows are copied
// by the global-to-LDS DMA (16 bytes per lane, no registers held): LDS slot
// u of the copy fetches the global chunk that belongs there. A block of
// zeros follows the rows: lanes past a row's last block read it, with a
// zero scale, and add exact zeros.
typedef __attribute__((address_space(3))) void* lds_ptr;

__device__ __forceinline__ void dma_slot(const float* src, int u0, int u, float* dst) {
  const int blk = u >> 3, c = (u & 7) ^ (blk & 7);
  __builtin_amdgcn_global_load_lds((const void*)(src + blk * 32 + c * 4), (lds_ptr)(dst + u0 * 4), 16, 0, 0);
}

// n floats (n % 32 == 0): the first NI * NT / 4 ... slots by NI unrolled
// instructions per wave (a loop would leave the compiler unable to count
// the loads issued after it), the rest, with LOOP only, by a loop.
template <int NT, int NI, bool LOOP>
__device__ __forceinline__ void dma_rows(const float* src, int n, float* dst) {
  const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
  const int slots = n / 4;
#pragma unroll
  for (int i = 0; i < NI; i++) {
    const int u0 = wave * WAVE + i * NT, u = u0 + lane;
    if (u < slots) dma_slot(src, u0, u, dst);  // inactive lanes write nothing
  }
  if (LOOP) {
    for (int u0 = wave * WAVE + NI * NT; u0 < slots; u0 += NT) {
      const int u = u0 + lane;
      if (u < slots) dma_slot(src, u0, u, dst);
    }
  }
}

// Block b of the row at `row` (or the zero block for b >= nb): base and
// chunk swizzle. The swizzle follows the block's index in the whole DMA
// copy: row_blocks = the blocks of the rows before this one.
__device__ __forceinline__ const float* xblock(const float* row, const float* zero, int b, int nb,
                                               int row_blocks, int& bm) {
  bm = b < nb ? ((row_blocks + b) & 7) : 0;
  return b < nb ? row + b * 32 : zero;
}

// Sum over the 32 lanes of a half-wave, the same in each of them.
__device__ __forceinline__ float half_sum(float v) {
#pragma unroll
  for (int off = 16; off >= 1; off >>= 1) v += __shfl_xor(v, off, WAVE);
  return v;
}

// One pass of a half-wave over blocks b0 + hl + 32 i (i < kSteps) of a row:
// codes and scale bytes in registers. Blocks past the row load the row's
// last block; the dot product gives them scale 0 and the zero block of the
// activation row. Nothing here uses a loaded value (code between these
// loads and the block barrier must not wait for them).
struct RowLoad {
  uint4 q[kSteps];
  uint8_t sc[kSteps];  // E8M0 byte (used only where the block lies in the row)
};

__device__ __forceinline__ void row_load(const uint8_t* blocks, const uint8_t* scales, size_t row,
                                         int nb, int b0, int hl, RowLoad& r) {
  const uint8_t* bq = blocks + row * (size_t)nb * 16;
  const uint8_t* bs = scales + row * (size_t)nb;
#pragma unroll
  for (int i = 0; i < kSteps; i++) {
    const int b = b0 + hl + 32 * i, bc = min(b, nb - 1);
    r.q[i] = load_nt_u4(bq + (size_t)bc * 16);
    r.sc[i] = bs[bc];
  }
}

// Materialises v[] in registers here: the products of a step cannot be
// deferred to the end of the kernel (the compiler would otherwise sink them
// and keep every activation read of the pass live at once).
template <int N>
__device__ __forceinline__ void pin_values(float (&v)[N]) {
#pragma unroll
  for (int i = 0; i < N; i++) asm volatile("" : "+v"(v[i]));
}

// acc[r] += block `st` of rows r < NR (codes q, scale sc) . the activation
// block at xb (chunk swizzle bm); each 8-value slice is read from LDS once
// for all rows.
// Per row the products are accumulated in element order.
template <int NR>
__device__ __forceinline__ void rows_block_dot(const RowLoad* rl, int st, const float* xb, int bm, bool in_row,
                                               float* acc) {
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const float4 xa = *(const float4*)(xb + (((2 * i) ^ bm) << 2));
    const float4 xc = *(const float4*)(xb + (((2 * i + 1) ^ bm) << 2));
#pragma unroll
    for (int r = 0; r < NR; r++) {
      const uint4 q = rl[r].q[st];
      const uint32_t w = i == 0 ? q.x : i == 1 ? q.y : i == 2 ? q.z : q.w;
      // scale 0 past the row, without a branch
      const float sc = __uint_as_float(__float_as_uint(e8m0_scale(rl[r].sc[st])) & (0u - (uint32_t)in_row));
      const float2v v0 = fp4_pair<0>(w, sc), v1 = fp4_pair<1>(w, sc);
      const float2v v2 = fp4_pair<2>(w, sc), v3 = fp4_pair<3>(w, sc);
      float a = acc[r];
      a = fmaf(v0.x, xa.x, a);
      a = fmaf(v0.y, xa.y, a);
      a = fmaf(v1.x, xa.z, a);
      a = fmaf(v1.y, xa.w, a);
      a = fmaf(v2.x, xc.x, a);
      a = fmaf(v2.y, xc.y, a);
      a = fmaf(v3.x, xc.z, a);
      a = fmaf(v3.y, xc.w, a);
      acc[r] = a;
    }
  }
}

// Waits until at most LOADS vector-memory operations are in flight (63 at
// most, the counter's range): with the activation DMA issued before LOADS
// weight loads (one code and one scale load per step and row), that
// completes the DMA.
template <int LOADS>
__device__ __forceinline__ void wait_dma_behind() {
  constexpr int N = LOADS < 63 ? LOADS : 63;
  __builtin_amdgcn_sched_barrier(0);  // no use of a weight load may be scheduled above this wait
  // s_waitcnt encoding (gfx9): vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] << 14
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Top-k of one token's router logits (E <= 64, one per lane) with the
// semantics of route_kernel's selection: each round takes the largest
// untaken logit, ties to the lowest expert id, NaN never selected unless it
// is the first untaken expert (a sequential scan starting from it would
// keep it); -inf only when nothing larger is left (the first untaken).
// Lane j < k ends with the j-th pick and its weight e^(l_j - l_0) / sum,
// the sum over the picks in pick order. Whole wave, uniform control flow.
__device__ __forceinline__ void topk_lanes(const float* lg, int E, int k, int& mine, float& wmine) {
  const int lane = threadIdx.x % WAVE;
  const float v = lane < E ? lg[lane] : -INFINITY;
  bool taken = false;
  int top = 0;
  mine = 0;
  for (int j = 0; j < k; j++) {
    const int first = __ffsll((unsigned long long)__ballot(lane < E && !taken)) - 1;  // k <= E: one is left
    const bool cand = lane < E && !taken && v > -INFINITY;
    int pick = first;
    if (__ballot(cand)) {
      const float M = wave_peak(cand ? v : -INFINITY);
      pick = __ffsll((unsigned long long)__ballot(cand && v == M)) - 1;
    }
    const float fv = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), first));
    if (fv != fv) pick = first;
    if (j == 0) top = pick;
    if (lane == j) mine = pick;
    if (lane == pick) taken = true;
  }
  const float lt = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), top));
  const float lm = __shfl(v, mine, WAVE);
  const float ev = lane < k ? expf(lm - lt) : 0.0f;
  float sum = 0.0f;
  for (int j = 0; j < k; j++) sum += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(ev), j));
  wmine = ev / sum;
}

// Router + top-k + softmax, one block of kRouteThreads per token: the
// activation row goes to LDS by DMA, then each wave issues every 128-bit
// weight load of its first kRouteE experts before any is used (further
// experts, for E > kRouteWaves * kRouteE, follow in a loop); wave 0 then
// selects. Measured at the MXFP4 MoE shape (256 tokens, 32 experts,
// d = 2880): 14.4 us with non-temporal weight loads, each row chunk read
// from LDS once per expert and every block starting at expert 0; 8.4 us
// with cached loads, one LDS read per chunk and the expert groups rotated
// by block. Two or more tokens per block (the weights applied to each row)
// spill registers and took 18-24 us.
constexpr int kRouteThreads = 512;
constexpr int kRouteWaves = kRouteThreads / WAVE;
constexpr int kRouteE = 4;     // experts per wave per pass
constexpr int kRouteLd = 6;    // 8-value chunks per lane per expert per pass
constexpr int kRouteDma = 4;   // unrolled DMA instructions per wave: d <= 8192

// Plain (cached) loads: every block reads the same router rows.
__device__ __forceinline__ void route_load(const uint16_t* router, int E, int d, int e0, int c0, int lane,
                                           uint4 (&w)[kRouteE][kRouteLd]) {
  const int chunks = d / 8;
#pragma unroll
  for (int i = 0; i < kRouteE; i++) {
    const uint16_t* wr = router + (size_t)min(e0 + i, E - 1) * d;
#pragma unroll
    for (int u = 0; u < kRouteLd; u++) w[i][u] = *(const uint4*)(wr + min(c0 + u * WAVE + lane, chunks - 1) * 8);
  }
}

// Each 8-value chunk of the row is read from LDS once for the wave's
// kRouteE experts; logit i still sums its chunks in order u = 0, 1, ...
__device__ __forceinline__ void route_dot(const uint4 (&w)[kRouteE][kRouteLd], const float* xs, int chunks,
                                          int c0, int lane, float (&acc)[kRouteE]) {
#pragma unroll
  for (int u = 0; u < kRouteLd; u++) {
    const int c = c0 + u * WAVE + lane;
    if (c < chunks) {
      const float4 xa = *(const float4*)(xs + c * 8), xb = *(const float4*)(xs + c * 8 + 4);
#pragma unroll
      for (int i = 0; i < kRouteE; i++) acc[i] = dot8(w[i][u], xa, xb, acc[i]);
    }
  }
}

template <bool LANE_E>
__global__ __launch_bounds__(kRouteThreads) void route_kernel(const float* xn, const uint16_t* router, int E,
                                                              int d, int k, int* sel, float* sel_w) {
  extern __shared__ __attribute__((aligned(16))) float sm[];
  float* xs = sm;      // [d]
  float* lg = sm + d;  // [E]
  const int t = blockIdx.x, lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  {
    const float* xrow = xn + (size_t)t * d;
#pragma unroll
    for (int i = 0; i < kRouteDma; i++) {
      const int u0 = wave * WAVE + i * kRouteThreads, u = u0 + lane;
      if (u < d / 4)  // inactive lanes write nothing
        __builtin_amdgcn_global_load_lds((const void*)(xrow + u * 4), (lds_ptr)(xs + u0 * 4), 16, 0, 0);
    }
  }
  const int chunks = d / 8;
  uint4 w[kRouteE][kRouteLd];
  // expert groups rotated by block, so that the blocks of an XCD do not all
  // request the same router rows at once
  const int g0 = (wave + (int)blockIdx.x) % kRouteWaves * kRouteE;
  route_load(router, E, d, g0, 0, lane, w);  // (clamped rows for a wave without experts)
  wait_dma_behind<kRouteE * kRouteLd>();
  __syncthreads();
  for (int e0 = g0; e0 < E; e0 += kRouteWaves * kRouteE) {
    float acc[kRouteE];
#pragma unroll
    for (int i = 0; i < kRouteE; i++) acc[i] = 0.0f;
    for (int c0 = 0; c0 < chunks; c0 += kRouteLd * WAVE) {
      if (e0 != g0 || c0 != 0) route_load(router, E, d, e0, c0, lane, w);
      route_dot(w, xs, chunks, c0, lane, acc);
    }
#pragma unroll
    for (int i = 0; i < kRouteE; i++) {
      const float v = wave_sum(acc[i]);
      if (lane == 0 && e0 + i < E) lg[e0 + i] = v;
    }
  }
  __syncthreads();
  if (LANE_E) {  // E <= 64: one expert per lane
    if (wave == 0) {
      int mine;
      float wm;
      topk_lanes(lg, E, k, mine, wm);
      if (lane < k) {
        sel[t * k + lane] = mine;
        sel_w[t * k + lane] = wm;
      }
    }
  } else if (wave == 0) {
    // k rounds of a wave-wide selection with the semantics of a sequential
    // scan over the experts not yet taken: start from the first, replace
    // on strictly greater (ties keep the lower id; a NaN first candidate
    // stays, later NaNs never win). Lane l holds experts l + 64 m; lane j
    // keeps the j-th pick.
    constexpr int kMaxPer = 1024 / WAVE;
    unsigned taken = 0;  // bit m: expert lane + 64 m taken
    int mine = 0, top = 0;
    for (int j = 0; j < k; j++) {
      int first = 0x7fffffff, bi = 0x7fffffff;
      float bv = -INFINITY;
#pragma unroll
      for (int m = 0; m < kMaxPer; m++) {
        const int e = lane + WAVE * m;
        if (e < E && !((taken >> m) & 1u)) {
          first = min(first, e);
          const float v = lg[e];
          if (v > bv || (v == bv && e < bi)) {
            bv = v;
            bi = e;
          }
        }
      }
#pragma unroll
      for (int off = 32; off >= 1; off >>= 1) {
        first = min(first, __shfl_xor(first, off, WAVE));
        const float ov = __shfl_xor(bv, off, WAVE);
        const int oi = __shfl_xor(bi, off, WAVE);
        if (ov > bv || (ov == bv && oi < bi)) {
          bv = ov;
          bi = oi;
        }
      }
      const float fv = lg[first];
      const int pick = (fv != fv || bi == 0x7fffffff) ? first : bi;
      if (j == 0) top = pick;
      if (lane == j) mine = pick;
      if (pick % WAVE == lane) taken |= 1u << (pick / WAVE);
    }
    // softmax over the k picks: e^(l_j - l_0), summed in pick order
    const float v = lane < k ? expf(lg[mine] - lg[top]) : 0.0f;
    float sum = 0.0f;
    for (int j = 0; j < k; j++) sum += __shfl(v, j, WAVE);
    if (lane < k) {
      sel[t * k + lane] = mine;
      sel_w[t * k + lane] = v / sum;
    }
  }
}

// Decode router (one token): block b computes the logits of experts
// 4b .. 4b+3, one per wavefront, each from the RMSNorm of the residual row
// formed in the block (the row and the norm weights are loaded before the
// router rows, which are all in flight before the first is used); block 0
// also writes the normalised row for the expert kernels. Logit e is the
// dot product in the lane order of route_kernel, summed across the wave by
// DPP.
constexpr int kRlXF = 8;   // float4 of the row per thread: d <= 8192
constexpr int kRlLd = 16;  // 8-value router chunks per lane: d <= 8192

__global__ __launch_bounds__(256) void route_logits_kernel(const float* x, const uint16_t* nw, float eps,
                                                           const uint16_t* router, int E, int d, float* logits,
                                                           float* xn) {
  extern __shared__ __attribute__((aligned(16))) float xs[];  // [d]
  __shared__ float red[4];
  const int lane = threadIdx.x % WAVE, wave = __builtin_amdgcn_readfirstlane(threadIdx.x / WAVE);
  const int e = blockIdx.x * 4 + wave;
  const int chunks = d / 8;
  float4 xv[kRlXF];
  uint2 nv[kRlXF];
#pragma unroll
  for (int i = 0; i < kRlXF; i++) {
    const int k = min((int)threadIdx.x * 4 + i * 1024, d - 4);
    xv[i] = *(const float4*)(x + k);
    nv[i] = *(const uint2*)(nw + k);
  }
  uint4 w[kRlLd];
  const uint16_t* wr = router + (size_t)min(e, E - 1) * d;
#pragma unroll
  for (int u = 0; u < kRlLd; u++) w[u] = load_nt_u4(wr + min(u * WAVE + lane, chunks - 1) * 8);
  __builtin_amdgcn_sched_barrier(0);  // the router loads go out before the staging waits
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < kRlXF; i++) {
    if ((int)threadIdx.x * 4 + i * 1024 < d) {
      ss = fmaf(xv[i].x, xv[i].x, ss);
      ss = fmaf(xv[i].y, xv[i].y, ss);
      ss = fmaf(xv[i].z, xv[i].z, ss);
      ss = fmaf(xv[i].w, xv[i].w, ss);
    }
  }
  const float s = rms_scale(block_sum<256>(ss, red), d, eps);
#pragma unroll
  for (int i = 0; i < kRlXF; i++) {
    const int k = (int)threadIdx.x * 4 + i * 1024;
    if (k < d) {
      float4 o;
      o.x = (xv[i].x * s) * bf16_to_f32((uint16_t)(nv[i].x & 0xffffu));
      o.y = (xv[i].y * s) * bf16_to_f32((uint16_t)(nv[i].x >> 16));
      o.z = (xv[i].z * s) * bf16_to_f32((uint16_t)(nv[i].y & 0xffffu));
      o.w = (xv[i].w * s) * bf16_to_f32((uint16_t)(nv[i].y >> 16));
      *(float4*)(xs + k) = o;
      if (blockIdx.x == 0) *(float4*)(xn + k) = o;
    }
  }
  __syncthreads();
  float acc = 0.0f;
#pragma unroll
  for (int u = 0; u < kRlLd; u++) {
    const int c = u * WAVE + lane;
    if (c < chunks) acc = dot8(w[u], *(const float4*)(xs + c * 8), *(const float4*)(xs + c * 8 + 4), acc);
  }
  acc = wave_total(acc);
  if (lane == 0 && e < E) logits[e] = acc;
}

// act[s][h] = silu(gate_e[h] . x_s) * (up_e[h] . x_s), slot s = (token, j):
// block (row group, slot); each half-wave takes kGuRows rows of both
// matrices. Order: expert id and activation loads, then every weight load
// of the first pass, then the activation row into LDS.
__device__ __forceinline__ void gu_load(const MoeGemvParams& p, int e, int r0, int nb, int b0, int hl,
                                        RowLoad (&ld)[2 * kGuRows]) {
#pragma unroll
  for (int r = 0; r < kGuRows; r++) {
    const size_t row = (size_t)e * p.N + min(r0 + r, p.N - 1);
    row_load(p.blocks, p.scales, row, nb, b0, hl, ld[r]);
    row_load(p.blocks2, p.scales2, row, nb, b0, hl, ld[kGuRows + r]);
  }
}

__device__ __forceinline__ void gu_dot(const RowLoad (&ld)[2 * kGuRows], const float* xs, const float* zero,
                                       int nb, int b0, int hl, float (&acc)[2 * kGuRows]) {
#pragma unroll
  for (int st = 0; st < kSteps; st++) {
    int bm;
    const int b = b0 + hl + 32 * st;
    const float* xb = xblock(xs, zero, b, nb, 0, bm);
    rows_block_dot<2 * kGuRows>(ld, st, xb, bm, b < nb, acc);
    pin_values<2 * kGuRows>(acc);
  }
}


// LOOP: rows longer than one pass (K > 32 * 32 * kSteps) take more passes
// (kept out of the one-pass kernel, whose registers it would share).
constexpr int kGuDma = 4;    // unrolled DMA instructions per wave: K <= 4096 without LOOP
constexpr int kDownDma = 12; // k * K <= 12288 without LOOP
template <bool LOOP>
__global__ __launch_bounds__(kThreads) void swiglu_kernel(MoeGemvParams p) {
  extern __shared__ __attribute__((aligned(16))) float xs[];  // [K] swizzled, then 32 zeros
  const int slot = blockIdx.y, lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  const int half = wave * 2 + lane / 32, hl = lane % 32;
  dma_rows<kThreads, kGuDma, LOOP>(p.x + (size_t)(slot / p.topk) * p.K, p.K, xs);
  int e;
  if (p.logits) {  // decode: this slot's expert from the router logits
    int mine;
    float wm;
    topk_lanes(p.logits + (size_t)(slot / p.topk) * p.E, p.E, p.topk, mine, wm);
    e = __builtin_amdgcn_readlane(mine, slot % p.topk);
  } else {
    e = p.expert[slot];
  }
  const int nb = p.K / 32;
  const int r0 = (blockIdx.x * kHalves + half) * kGuRows;
  float acc[2 * kGuRows];  // gate rows, then up rows
#pragma unroll
  for (int r = 0; r < 2 * kGuRows; r++) acc[r] = 0.0f;
  RowLoad ld[2 * kGuRows];
  gu_load(p, e, r0, nb, 0, hl, ld);
  float* zero = xs + p.K;
  if (threadIdx.x < 32) zero[threadIdx.x] = 0.0f;
  wait_dma_behind<2 * 2 * kGuRows * kSteps>();
  __syncthreads();
  gu_dot(ld, xs, zero, nb, 0, hl, acc);
  if (LOOP) {
    for (int b0 = 32 * kSteps; b0 < nb; b0 += 32 * kSteps) {
      RowLoad ln[2 * kGuRows];
      gu_load(p, e, r0, nb, b0, hl, ln);
      gu_dot(ln, xs, zero, nb, b0, hl, acc);
    }
  }
#pragma unroll
  for (int r = 0; r < kGuRows; r++) {
    const float gs = half_sum(acc[r]), us = half_sum(acc[kGuRows + r]);
    if (hl == 0 && r0 + r < p.N) p.y[(size_t)slot * p.N + r0 + r] = silu_mul(gs, us);
  }
}

// y[t][n] += sum_j fmaf order of w_j * (down_e_j[n] . act[t*k + j]):
// block (row group, token); each half-wave takes kDownRows rows, for every
// slot of the token, all their loads of a pass in flight at once (the
// activation DMA goes first).
template <int KMAX>
__device__ __forceinline__ void down_load(const MoeGemvParams& p, const int (&e)[KMAX], int n0, int nb, int b0,
                                          int hl, RowLoad (&ld)[kDownRows * KMAX]) {
#pragma unroll
  for (int r = 0; r < kDownRows; r++)
#pragma unroll
    for (int j = 0; j < KMAX; j++)
      row_load(p.blocks, p.scales, (size_t)e[j] * p.N + min(n0 + r, p.N - 1), nb, b0, hl, ld[r * KMAX + j]);
}

// Slots past k (KMAX > k) repeat slot k - 1; their sums are dropped.
template <int KMAX>
__device__ __forceinline__ void down_dot(const RowLoad (&ld)[kDownRows * KMAX], const float* as, const float* zero,
                                         int k, int K, int nb, int b0, int hl, float (&dot)[kDownRows * KMAX]) {
#pragma unroll
  for (int st = 0; st < kSteps; st++) {
#pragma unroll
    for (int j = 0; j < KMAX; j++) {
      int bm;
      const int b = b0 + hl + 32 * st;
      const int row = min(j, k - 1);
      const float* xb = xblock(as + row * K, zero, b, nb, row * nb, bm);
#pragma unroll
      for (int r = 0; r < kDownRows; r++)
        rows_block_dot<1>(&ld[r * KMAX + j], st, xb, bm, b < nb, &dot[r * KMAX + j]);
    }
    pin_values<kDownRows * KMAX>(dot);
  }
}

template <int KMAX, bool LOOP>
__global__ __launch_bounds__(kThreads) void down_kernel(MoeGemvParams p) {
  extern __shared__ __attribute__((aligned(16))) float as[];  // [k][K] swizzled, then 32 zeros
  const int k = p.topk;
  const int t = blockIdx.y, lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  const int half = wave * 2 + lane / 32, hl = lane % 32;
  dma_rows<kThreads, kDownDma, LOOP>(p.x + (size_t)t * k * p.K, k * p.K, as);
  int e[KMAX];
  float wt[KMAX];
  if (p.logits) {  // decode: the token's experts and weights from the router logits
    int mine;
    float wm;
    topk_lanes(p.logits + (size_t)t * p.E, p.E, k, mine, wm);
#pragma unroll
    for (int j = 0; j < KMAX; j++) {
      e[j] = __builtin_amdgcn_readlane(mine, min(j, k - 1));
      wt[j] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(wm), min(j, k - 1)));
    }
  } else {
#pragma unroll
    for (int j = 0; j < KMAX; j++) {
      e[j] = p.expert[t * k + min(j, k - 1)];
      wt[j] = p.weight[t * k + min(j, k - 1)];
    }
  }
  const int nb = p.K / 32;
  const int n0 = (blockIdx.x * kHalves + half) * kDownRows;
  float dot[kDownRows * KMAX];
#pragma unroll
  for (int i = 0; i < kDownRows * KMAX; i++) dot[i] = 0.0f;
  RowLoad ld[kDownRows * KMAX];  // row r, slot j at r * KMAX + j
  down_load<KMAX>(p, e, n0, nb, 0, hl, ld);
  float* zero = as + k * p.K;
  if (threadIdx.x < 32) zero[threadIdx.x] = 0.0f;
  wait_dma_behind<2 * kDownRows * KMAX * kSteps>();
  __syncthreads();
  down_dot<KMAX>(ld, as, zero, k, p.K, nb, 0, hl, dot);
  if (LOOP) {
    for (int b0 = 32 * kSteps; b0 < nb; b0 += 32 * kSteps) {
      RowLoad ln[kDownRows * KMAX];
      down_load<KMAX>(p, e, n0, nb, b0, hl, ln);
      down_dot<KMAX>(ln, as, zero, k, p.K, nb, b0, hl, dot);
    }
  }
#pragma unroll
  for (int r = 0; r < kDownRows; r++) {
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < KMAX; j++)
      if (j < k) acc = fmaf(wt[j], half_sum(dot[r * KMAX + j]), acc);
    const int n = n0 + r;
    if (hl == 0 && n < p.N) p.y[(size_t)t * p.N + n] += acc;
  }
}

// The decode of mx_block_dot, written out: out[32 b + i] = value i of block b.
__global__ void mxfp4_decode_kernel(const uint8_t* codes, const uint8_t* scales, int nblocks, float* out,
                                    int bf16_tiles) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= nblocks) return;
  const uint4 q = *(const uint4*)(codes + (size_t)b * 16);
  const float sc = e8m0_scale(scales[b]);
  const uint32_t w[4] = {q.x, q.y, q.z, q.w};
  float* o = out + (size_t)b * 32;
  if (bf16_tiles) {  // the grouped prefill GEMM's conversion, widened back
    uint32_t t[16];
    fp4_block_bf16(w, sc, t);
#pragma unroll
    for (int j = 0; j < 16; j++) {
      o[2 * j] = __uint_as_float(t[j] << 16);
      o[2 * j + 1] = __uint_as_float(t[j] & 0xFFFF0000u);
    }
    return;
  }
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const float2v v0 = fp4_pair<0>(w[i], sc), v1 = fp4_pair<1>(w[i], sc);
    const float2v v2 = fp4_pair<2>(w[i], sc), v3 = fp4_pair<3>(w[i], sc);
    o[8 * i + 0] = v0.x;
    o[8 * i + 1] = v0.y;
    o[8 * i + 2] = v1.x;
    o[8 * i + 3] = v1.y;
    o[8 * i + 4] = v2.x;
    o[8 * i + 5] = v2.y;
    o[8 * i + 6] = v3.x;
    o[8 * i + 7] = v3.y;
  }
}

// ------------------------------------------------- prefill: grouped GEMM --
//
// Slots s = (token, j) are grouped by expert (moe_group: counting sort,
// stable in slot order), then each expert's slots go through an MFMA GEMM
// whose B operand is the expert's MXFP4 matrix, decoded into LDS as bf16
// (exact: an E2M1 value times a power of two has at most two significant
// bits). The A rows (fp32 activations) are split into bf16 hi + lo planes
// on the way into LDS, as the dense prefill GEMM does, so both products are
// exact in the fp32 accumulator. Tile: 32 slots x 64 weight rows (x2 for the
// gate/up pair), K steps of 32 (one MXFP4 block per row), 4 waves each
// owning 16 weight rows; LDS double-buffered, the next step's global loads
// in registers while the current step multiplies.

constexpr int GBM = 32, GBN = 64, GBK = 32, GLD = 40;  // LDS row stride (bf16)

// The same with the expert ids staged in LDS once (n <= kGroup2MaxN, E <=
// 64): wave w takes a contiguous run of slots, 64 ids at a time in
// registers, and lane e keeps expert e's count (one ballot per expert);
// lane e of wave 0 turns the counts into each run's first position within
// expert e (runs in order, so the slots of an expert stay increasing), and
// each wave scatters its run. group_kernel below re-reads the ids for
// every expert in dependent steps.
constexpr int kGroup2MaxN = 32768;
__global__ __launch_bounds__(1024) void group2_kernel(const int* sel, int n, int E, int* offs, int* order) {
  extern __shared__ int ids[];       // [n]
  __shared__ int cnt[16][WAVE];      // hits per (wave run, expert), then first positions
  const int lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  for (int i = threadIdx.x; i < n; i += 1024) ids[i] = sel[i];
  __syncthreads();
  const int groups = (n + WAVE - 1) / WAVE, per = (groups + 15) / 16;
  const int b0 = wave * per * WAVE, b1 = min(n, (wave + 1) * per * WAVE);
  int mine = 0;  // lane e: hits of expert e in this wave's run
  for (int b = b0; b < b1; b += WAVE) {
    const int v = b + lane < b1 ? ids[b + lane] : -1;
    for (int e = 0; e < E; e++) {
      const int c = __popcll(__ballot(v == e));
      if (lane == e) mine += c;
    }
  }
  if (lane < E) cnt[wave][lane] = mine;
  __syncthreads();
  if (wave == 0) {
    int tot = 0;
    if (lane < E)
      for (int w = 0; w < 16; w++) tot += cnt[w][lane];
    // exclusive prefix over experts (lanes)
    int inc = tot;
    for (int off = 1; off < WAVE; off <<= 1) {
      const int y = __shfl_up(inc, off, WAVE);
      if (lane >= off) inc += y;
    }
    int run = inc - tot;
    if (lane < E) {
      offs[lane] = run;
      for (int w = 0; w < 16; w++) {
        const int c = cnt[w][lane];
        cnt[w][lane] = run;
        run += c;
      }
    }
    if (lane == E - 1) offs[E] = inc;
  }
  __syncthreads();
  int next = lane < E ? cnt[wave][lane] : 0;  // lane e: next position of expert e
  for (int b = b0; b < b1; b += WAVE) {
    const int v = b + lane < b1 ? ids[b + lane] : -1;
    for (int e = 0; e < E; e++) {
      const unsigned long long m = __ballot(v == e);
      const int pos = __builtin_amdgcn_readlane(next, e);
      if (v == e) order[pos + __popcll(m & ((1ull << lane) - 1))] = b + lane;
      if (lane == e) next += __popcll(m);
    }
  }
}

// order[offs[e] .. offs[e+1]) = the slots routed to expert e, increasing.
__global__ __launch_bounds__(1024) void group_kernel(const int* sel, int n, int E, int* offs, int* order) {
  extern __shared__ int cnt[];  // [E + 1]
  const int lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE, nw = blockDim.x / WAVE;
  for (int e = wave; e < E; e += nw) {
    int c = 0;
    for (int b = 0; b < n; b += WAVE) {
      const bool hit = b + lane < n && sel[b + lane] == e;
      c += __popcll(__ballot(hit));
    }
    if (lane == 0) cnt[e] = c;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    int run = 0;
    for (int e = 0; e < E; e++) {
      const int c = cnt[e];
      cnt[e] = run;
      offs[e] = run;
      run += c;
    }
    offs[E] = run;
  }
  __syncthreads();
  for (int e = wave; e < E; e += nw) {
    int pos = cnt[e];
    for (int b = 0; b < n; b += WAVE) {
      const bool hit = b + lane < n && sel[b + lane] == e;
      const unsigned long long m = __ballot(hit);
      if (hit) order[pos + __popcll(m & ((1ull << lane) - 1))] = b + lane;
      pos += __popcll(m);
    }
  }
}

template <bool DUAL>
__global__ __launch_bounds__(256) void group_gemm_kernel(MoeGemmParams p) {
  constexpr int NM = DUAL ? 2 : 1;
  __shared__ __attribute__((aligned(16))) uint16_t ahi[2][GBM * GLD], alo[2][GBM * GLD];
  __shared__ __attribute__((aligned(16))) uint16_t bw[2][NM][GBN * GLD];
  __shared__ int tile_info[2];
  const int tid = threadIdx.x, lane = tid % WAVE, wave = tid / WAVE;
  // Which expert and which 32-slot tile of it this block computes.
  if (wave == 0) {
    int e_found = -1, m0 = 0, base = 0;
    for (int e0 = 0; e0 < p.E && e_found < 0; e0 += WAVE) {
      const int e = e0 + lane;
      const int c = e < p.E ? p.offs[e + 1] - p.offs[e] : 0;
      int tiles = (c + GBM - 1) / GBM, incl = tiles;
#pragma unroll
      for (int off = 1; off < WAVE; off <<= 1) {
        const int v = __shfl_up(incl, off, WAVE);
        if (lane >= off) incl += v;
      }
      const int excl = base + incl - tiles;
      const bool mine = (int)blockIdx.x >= excl && (int)blockIdx.x < excl + tiles;
      const unsigned long long m = __ballot(mine);
      if (m) {
        const int src = __ffsll((long long)m) - 1;
        e_found = __shfl(e0 + lane, src, WAVE);
        m0 = ((int)blockIdx.x - __shfl(excl, src, WAVE)) * GBM;
      }
      base += __shfl(incl, WAVE - 1, WAVE);
    }
    if (lane == 0) {
      tile_info[0] = e_found;
      tile_info[1] = m0;
    }
  }
  __syncthreads();
  const int e = tile_info[0], m0 = tile_info[1];
  if (e < 0) return;  // past the last tile (the grid is an upper bound)
  const int cnt = p.offs[e + 1] - p.offs[e];
  const int n0 = blockIdx.y * GBN;
  const int K = p.K, nb = K / 32;

  // loader roles: A: row ar, 4 values at ac; B: matrix bm, row br, half bh
  const int ar = tid / 8, ac = (tid % 8) * 4;
  const bool a_ok = m0 + ar < cnt;
  const int slot = a_ok ? p.order[p.offs[e] + m0 + ar] : 0;
  const float* arow = p.a + (size_t)(p.a_per_token ? slot / p.topk : slot) * K;
  const int bm = tid / 128, br = (tid % 128) / 2, bh = tid % 2;
  const bool b_ok = bm < NM;
  const size_t brow = (size_t)e * p.N + min(n0 + br, p.N - 1);
  const uint8_t* bq = (bm == 0 ? p.blocks : p.blocks2) + brow * (size_t)nb * 16 + bh * 8;
  const uint8_t* bsc = (bm == 0 ? p.scales : p.scales2) + brow * (size_t)nb;

  float4 ra;
  uint2 rq;
  unsigned rs;
  auto fetch = [&](int kb) {
    ra = a_ok ? *(const float4*)(arow + kb * GBK + ac) : make_float4(0.f, 0.f, 0.f, 0.f);
    if (b_ok) {
      rq = *(const uint2*)(bq + (size_t)kb * 16);
      rs = bsc[kb];
    }
  };
  auto stash = [&](int buf) {
    const float av[4] = {ra.x, ra.y, ra.z, ra.w};
    uint16_t h[4], l[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      h[i] = f32_to_bf16_rne(av[i]);
      l[i] = f32_to_bf16_rne(av[i] - bf16_to_f32(h[i]));
    }
    *(uint2*)(ahi[buf] + ar * GLD + ac) = make_uint2(h[0] | ((unsigned)h[1] << 16), h[2] | ((unsigned)h[3] << 16));
    *(uint2*)(alo[buf] + ar * GLD + ac) = make_uint2(l[0] | ((unsigned)l[1] << 16), l[2] | ((unsigned)l[3] << 16));
    if (b_ok) {
      const float sc = e8m0_scale(rs);
      const uint32_t w[2] = {rq.x, rq.y};
      unsigned out[8];
#pragma unroll
      for (int i = 0; i < 2; i++) {
        const float2v v0 = fp4_pair<0>(w[i], sc), v1 = fp4_pair<1>(w[i], sc);
        const float2v v2 = fp4_pair<2>(w[i], sc), v3 = fp4_pair<3>(w[i], sc);
        out[4 * i + 0] = (__float_as_uint(v0.x) >> 16) | (__float_as_uint(v0.y) & 0xFFFF0000u);
        out[4 * i + 1] = (__float_as_uint(v1.x) >> 16) | (__float_as_uint(v1.y) & 0xFFFF0000u);
        out[4 * i + 2] = (__float_as_uint(v2.x) >> 16) | (__float_as_uint(v2.y) & 0xFFFF0000u);
        out[4 * i + 3] = (__float_as_uint(v3.x) >> 16) | (__float_as_uint(v3.y) & 0xFFFF0000u);
      }
      uint4* dst = (uint4*)(bw[buf][bm] + br * GLD + bh * 16);
      dst[0] = make_uint4(out[0], out[1], out[2], out[3]);
      dst[1] = make_uint4(out[4], out[5], out[6], out[7]);
    }
  };

  f32x4 acc[NM][2];
#pragma unroll
  for (int m = 0; m < NM; m++) acc[m][0] = acc[m][1] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int fr = lane % 16, fk = (lane / 16) * 8;
  fetch(0);
  for (int kb = 0; kb < nb; kb++) {
    const int buf = kb & 1;
    stash(buf);
    __syncthreads();
    if (kb + 1 < nb) fetch(kb + 1);
    bf16x8 a_h[2], a_l[2], b[NM];
#pragma unroll
    for (int mi = 0; mi < 2; mi++) {
      a_h[mi] = *(const bf16x8*)(ahi[buf] + (mi * 16 + fr) * GLD + fk);
      a_l[mi] = *(const bf16x8*)(alo[buf] + (mi * 16 + fr) * GLD + fk);
    }
#pragma unroll
    for (int m = 0; m < NM; m++) b[m] = *(const bf16x8*)(bw[buf][m] + (wave * 16 + fr) * GLD + fk);
#pragma unroll
    for (int m = 0; m < NM; m++)
#pragma unroll
      for (int mi = 0; mi < 2; mi++) {
        acc[m][mi] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_h[mi], b[m], acc[m][mi], 0, 0, 0);
        acc[m][mi] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a_l[mi], b[m], acc[m][mi], 0, 0, 0);
      }
  }
  // lane holds C[4 (lane / 16) + i][lane % 16] of each 16 x 16 tile
  const int n = n0 + wave * 16 + lane % 16;
  if (n >= p.N) return;
#pragma unroll
  for (int mi = 0; mi < 2; mi++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int r = mi * 16 + (lane / 16) * 4 + i;
      if (m0 + r >= cnt) continue;
      const int s2 = p.order[p.offs[e] + m0 + r];
      p.y[(size_t)s2 * p.N + n] = DUAL ? silu_mul(acc[0][mi][i], acc[NM - 1][mi][i]) : acc[0][mi][i];
    }
}

// ------------------------------------- prefill: pipelined grouped GEMM --
//
// Same product as group_gemm_kernel, restructured for the memory system:
// * A (the slots' activation rows) comes pre-split into bf16 hi/lo planes in
//   expert order (moe_gather_split), so a tile's rows are contiguous and go
//   to LDS by the global-to-LDS DMA in 128-byte row segments (K steps of
//   64), 3-stage ring;
// * the MXFP4 code bytes of the tile's QBR weight rows (half gate, half up,
//   or QBR rows of one matrix; QBR x 32 bytes per step) go with the A rows
//   of the same step into the same slot of a 3-stage DMA ring; the rows'
//   E8M0 scales are DMA'd once per block and converted to fp32 a step ahead;
// * each wave converts the codes of its own weight rows straight into its
//   MFMA B operands (hardware FP4 conversion to packed bf16 pairs, exact),
//   so no decoded tile goes through LDS: BM slots (32, or 64 when the
//   experts average at least 24 slots, so that one tile covers most experts
//   and their weights stream once) x QBR rows x 64 K per step, 4 BM / 16
//   QFR MFMAs per wave (each wave: all BM slots x QFR 16-row fragments;
//   a 2 x 2 split of the waves, half the A stage each but twice the code
//   conversions, measured slower). Every wave reads the whole A stage, so wider blocks read A
//   less often per product: QBR = 256 takes 1.2x the time of 128 for twice
//   the work, but its grid of half as many blocks (at two per CU, 75 KiB of
//   LDS) leaves a partial last round at the 256-token prefill and loses
//   there (228 vs 193 us for the gate/up pair); it wins at 2048 tokens
//   (927 vs 1018 us). QBR = 128: ~50 KiB of LDS at K = 2880, three blocks
//   per CU.
// * the grid is laid out per XCD (see the kernel).
// Each step issues exactly QAI A + QBI code DMA instructions per wave
// (indexes past the last step are clamped to it and never read), so the
// wait before a step is a constant: the groups of the QNA - 2 later steps
// may stay in flight.
constexpr int QKS = 64, QBR = 128;  // K per step, weight rows per block
constexpr int QFR = QBR / 64;                  // 16-row B fragments per wave
constexpr int QBI = QBR / 128;                 // code DMA instructions per wave and step
constexpr int kXcds = 8;                      // XCDs of an MI355X (round-robin block dispatch)

__device__ __forceinline__ int wave_sum_int(int v) {
#pragma unroll
  for (int off = WAVE / 2; off >= 1; off >>= 1) v += __shfl_xor(v, off, WAVE);
  return v;
}
constexpr int QNA = 3, QNB = 3;              // A ring, code ring stages
template <int BM>
constexpr int q_ai() { return 2 * BM * QKS * 2 / 1024 / 4; }  // A DMA instructions per wave and step
constexpr int kQMaxNb = 256;                  // K / 32 <= 256 (scales per row)

// Scale bytes per run (one run per matrix): rows x nb, in whole 1 KiB DMA
// instructions so that the runs' tails never overlap.
__host__ __device__ constexpr int q_scale_run(int rows, int nb) { return (rows * nb + 1023) / 1024 * 1024; }

template <int BM>
struct QLds {
  static constexpr int a_stage = 2 * BM * QKS * 2;  // hi + lo rows of 128 bytes
  static constexpr int b_stage = QBR * 32;           // 2 code blocks per row
  static constexpr int a = 0;
  static constexpr int b = a + QNA * a_stage;
  static constexpr int info = b + QNB * b_stage;     // the tile lookup result
  static constexpr int fsc = info + 256;             // [2][QBR rows][2 blocks] fp32 scales of a step
  static constexpr int sc = (fsc + 2 * QBR * 2 * 4 + 1023) / 1024 * 1024;  // scales: QBR rows x nb bytes
};
static_assert(QNA == QNB, "one ring slot per step for the A rows and the codes");
static_assert(QLds<64>::sc + 2 * ((128 * 256 / 2 + 1023) / 1024 * 1024) <= 160 * 1024, "grouped GEMM LDS");

__device__ __forceinline__ int q_swz(int r) { return (r >> 1) & 7; }  // 128-byte rows

// LDS reads of DMA-written data use vector types: through HIP's uint4
// struct the compiler waits for every DMA in flight before the read (the
// explicit waits and barriers order the data).
typedef unsigned q_u32x4 __attribute__((ext_vector_type(4)));

// The tile of a grouped-GEMM block, found by one wavefront: tile_info =
// {expert or -1 past the last tile, first slot of the tile, column tile}.
// The (slot tile, column tile) grid is laid out per XCD (blocks are
// dispatched to the 8 XCDs round-robin by linear id): XCD x takes a
// contiguous run of the slot tiles (about an eighth of the experts) and
// walks the column tiles in its outer loop, so the A rows of its tiles
// stay in its L2 across column tiles and the slot tiles of one expert, run
// side by side, share each column tile's codes.
template <int BM>
__device__ void group_tile_lookup(const MoeGemmParams& p, int lane, int* tile_info) {
  // total slot tiles (experts in order, ceil(count / BM) each)
  int tr = 0;
  for (int e0 = 0; e0 < p.E; e0 += WAVE) {
    const int e = e0 + lane;
    const int c = e < p.E ? p.offs[e + 1] - p.offs[e] : 0;
    tr += wave_sum_int((c + BM - 1) / BM);
  }
  const int lin = (int)(blockIdx.x + blockIdx.y * gridDim.x);
  const int xcd = lin % kXcds, j = lin / kXcds, ny = (int)gridDim.y;
  const int lo = xcd * tr / kXcds, nt = (xcd + 1) * tr / kXcds - lo;
  int e_found = -1, m0 = 0, y = 0;
  if (nt > 0 && j < nt * ny) {
    y = j / nt;
    const int T = lo + j % nt;
    int base = 0;
    for (int e0 = 0; e0 < p.E && e_found < 0; e0 += WAVE) {
      const int e = e0 + lane;
      const int c = e < p.E ? p.offs[e + 1] - p.offs[e] : 0;
      int tiles = (c + BM - 1) / BM, incl = tiles;
#pragma unroll
      for (int off = 1; off < WAVE; off <<= 1) {
        const int v = __shfl_up(incl, off, WAVE);
        if (lane >= off) incl += v;
      }
      const int excl = base + incl - tiles;
      const unsigned long long m = __ballot(T >= excl && T < excl + tiles);
      if (m) {
        const int src = __ffsll((long long)m) - 1;
        e_found = __shfl(e0 + lane, src, WAVE);
        m0 = (T - __shfl(excl, src, WAVE)) * BM;
      }
      base += __shfl(incl, WAVE - 1, WAVE);
    }
  }
  if (lane == 0) {
    tile_info[0] = e_found;
    tile_info[1] = m0;
    tile_info[2] = y;
  }
}

// BM slots per block (32 or 64; 64 when experts average enough slots that
// one tile covers most of them, so each expert's weights stream once).
template <bool DUAL, int BM>
__global__ __launch_bounds__(256, 2) void group_gemm2_kernel(MoeGemmParams p) {
  using QL = QLds<BM>;
  constexpr int QAI = q_ai<BM>();
  constexpr int MS = BM / 16;  // 16-slot sub-tiles
  // one LDS object (a second one makes the compiler wait for every LDS DMA
  // before any LDS read)
  extern __shared__ __attribute__((aligned(1024))) unsigned char ql[];
  int* tile_info = (int*)(ql + QL::info);
  const int tid = threadIdx.x, lane = tid % WAVE, wave = tid / WAVE;
  if (wave == 0) group_tile_lookup<BM>(p, lane, tile_info);
  __syncthreads();
  const int e = tile_info[0], m0 = tile_info[1];
  if (e < 0) return;  // past the last tile (the grid is an upper bound)
  const int rbeg = p.offs[e], cnt = p.offs[e + 1] - rbeg;
  const int cols = DUAL ? QBR / 2 : QBR;  // output columns per block
  const int n0 = tile_info[2] * cols;
  const int K = p.K, nb = K / 32, nk = K / QKS;
  // 16-slot sub-tiles holding at least one slot of the expert: the others
  // are padding, whose A reads and products are skipped (wave-uniform, so
  // the MFMAs always run with every lane on)
  const int act = __builtin_amdgcn_readfirstlane(min(MS, (cnt - m0 + 15) / 16));

  // --- DMA sources (per lane) ---
  // A: instruction i (< QAI) of this wave covers stage rows 8 (QAI wave + i)
  // .., rows 0..BM-1 hi, BM..2 BM-1 lo; lane -> row + lane / 8, physical
  // chunk lane % 8.
  const uint16_t* asrc[QAI];
#pragma unroll
  for (int i = 0; i < QAI; i++) {
    const int row = 8 * (QAI * wave + i) + lane / 8;
    const int c = (lane % 8) ^ q_swz(row);
    const int r = row % BM;
    const int grow = rbeg + min(m0 + r, cnt - 1);  // rows past the tile load its last row
    const int srow = p.a_per_token ? p.order[grow] / p.topk : grow;
    asrc[i] = (row < BM ? p.a_hi : p.a_lo) + (size_t)srow * K + 8 * c;
  }
  // codes: instruction i of wave w covers weight rows 32 (QBI w + i) ..
  // + 31, lane -> row + lane / 2, block lane % 2 of the step
  const uint8_t* bsrc[QBI];
#pragma unroll
  for (int i = 0; i < QBI; i++) {
    const int br = 32 * (QBI * wave + i) + lane / 2;
    const bool up = DUAL && br >= QBR / 2;
    const int n = min(n0 + (DUAL ? br % (QBR / 2) : br), p.N - 1);
    bsrc[i] = (up ? p.blocks2 : p.blocks) + ((size_t)e * p.N + n) * nb * 16 + (lane % 2) * 16;
  }

  // scales of the block's rows: per matrix a contiguous run of rows x nb
  // bytes (16-byte aligned: the host checks N % 16 == 0), 1 KiB per
  // instruction; lanes past the run read in-bounds bytes that are not used
  {
    const int runs = DUAL ? 2 : 1, rows = QBR / runs;
    const int run = q_scale_run(rows, nb), ni = run / 1024;
    const size_t off0 = ((size_t)e * p.N + n0) * nb;
    const size_t limit = ((size_t)(e + 1) * p.N) * nb - 16;  // last 16-byte chunk of expert e's scales
    for (int rr = 0; rr < runs; rr++) {
      const uint8_t* sb = rr == 0 ? p.scales : p.scales2;
      for (int n = wave; n < ni; n += 4) {
        const size_t o = min(off0 + (size_t)n * 1024 + 16 * lane, limit);
        __builtin_amdgcn_global_load_lds((const void*)(sb + o), (lds_ptr)(ql + QL::sc + rr * run + n * 1024),
                                         16, 0, 0);
      }
    }
  }
  // B operands straight from the code stage: wave w takes QFR fragments of
  // 16 weight rows (DUAL: the gate and up rows of its QFR / 2 16-column
  // groups of the block's output columns; otherwise QFR 16-column groups of
  // one matrix). Lane
  // (g, c) = (lane / 16, lane % 16) takes, for MFMA k-step kk of a 64-value
  // step (= MX block kk of its row), values 8 g .. 8 g + 7: code bytes
  // 4 g .. 4 g + 3 of the block and the block's scale, converted in
  // registers. The A operand of lane (g, c): chunk 4 kk + g of its slot
  // row, the same K values.
  const int g = lane / 16, c = lane % 16;
  constexpr int HF = QFR / 2;  // DUAL: column groups per wave
  int brow[QFR];
#pragma unroll
  for (int f = 0; f < QFR; f++)
    brow[f] = DUAL ? (f < HF ? 16 * HF * wave + 16 * f + c : QBR / 2 + 16 * HF * wave + 16 * (f - HF) + c)
                   : 16 * QFR * wave + 16 * f + c;
  auto achunk = [&](const unsigned char* as, int r, int ch) -> bf16x8 {
    return *(const bf16x8*)(as + r * 128 + ((ch ^ q_swz(r)) << 4));
  };

  f32x4 acc[MS][QFR];  // [16-slot sub-tile][fragment]
#pragma unroll
  for (int i = 0; i < MS; i++)
#pragma unroll
    for (int f = 0; f < QFR; f++) acc[i][f] = f32x4{0.f, 0.f, 0.f, 0.f};

  // step t: A rows and codes into ring slot t % QNA (indexes past the last
  // step clamped to it: read, never used)
  auto issue_a = [&](int t) {
    const int tc = min(t, nk - 1);
    unsigned char* as = ql + QL::a + (t % QNA) * QL::a_stage;
#pragma unroll
    for (int i = 0; i < QAI; i++)
      __builtin_amdgcn_global_load_lds((const void*)(asrc[i] + tc * QKS),
                                       (lds_ptr)(as + (QAI * wave + i) * 1024), 16, 0, 0);
  };
  auto issue_b = [&](int t) {
    const int tc = min(t, nk - 1);
    unsigned char* bs = ql + QL::b + (t % QNB) * QL::b_stage;
#pragma unroll
    for (int i = 0; i < QBI; i++)
      __builtin_amdgcn_global_load_lds((const void*)(bsrc[i] + (size_t)tc * 32),
                                       (lds_ptr)(bs + (QBI * wave + i) * 1024), 16, 0, 0);
  };
  auto issue_group = [&](int t) {
    issue_a(t);
    issue_b(t);
  };
  // the codes of the first steps go out before the A rows, whose addresses
  // wait for the slot indices when A is read one row per token
#pragma unroll
  for (int t = 0; t < QNA - 1; t++) issue_b(t);
#pragma unroll
  for (int t = 0; t < QNA - 1; t++) issue_a(t);
  // the scales (a per-shape number of DMA instructions) and the first
  // groups: waited for here, so that the loop's waits are exact counts
  wait_dma_behind<0>();
  __syncthreads();
  // the E8M0 scales of a step as fp32 (row q / 2, block q % 2 for q = tid,
  // tid + 256, ..), a step ahead of their use
  float* fsc = (float*)(ql + QL::fsc);
  constexpr int NCS = 2 * QBR / 256;  // scales per thread and step
  int csrc[NCS];
#pragma unroll
  for (int i = 0; i < NCS; i++) {
    const int q = tid + 256 * i, crow = q / 2;
    csrc[i] = QL::sc + (DUAL ? (crow / (QBR / 2)) * q_scale_run(QBR / 2, nb) + (crow % (QBR / 2)) * nb
                               : crow * nb) + q % 2;
    fsc[q] = e8m0_scale(ql[csrc[i]]);
  }
  for (int kt = 0; kt < nk; kt++) {
    // this wave's scales and groups up to kt landed (the QNA - 2 later
    // groups may stay in flight); the barrier extends that to every wave's
    // and frees the slot of step kt - 1
    wait_dma_behind<(QAI + QBI) * (QNA - 2)>();
    __syncthreads();
    // every operand of step kt from LDS first, then the next group's DMA
    // (into the slot of step kt - 1)
    const unsigned char* as = ql + QL::a + (kt % QNA) * QL::a_stage;
    const unsigned char* bs = ql + QL::b + (kt % QNB) * QL::b_stage;
    unsigned w[QFR][2];  // [fragment][k-step]: 8 codes
    float sc[QFR][2];
#pragma unroll
    for (int f = 0; f < QFR; f++) {
      const float2v s2 = *(const float2v*)(fsc + (kt & 1) * 2 * QBR + 2 * brow[f]);
      sc[f][0] = s2[0];
      sc[f][1] = s2[1];
#pragma unroll
      for (int kk = 0; kk < 2; kk++) w[f][kk] = *(const unsigned*)(bs + brow[f] * 32 + kk * 16 + 4 * g);
    }
    if (kt + 1 < nk) {
#pragma unroll
      for (int i = 0; i < NCS; i++) fsc[((kt + 1) & 1) * 2 * QBR + tid + 256 * i] = e8m0_scale(ql[csrc[i] + 2 * (kt + 1)]);
    }
    bf16x8 ah[2][MS], al[2][MS];  // [k-step][16-slot sub-tile]
#pragma unroll
    for (int kk = 0; kk < 2; kk++)
#pragma unroll
      for (int mi = 0; mi < MS; mi++) {
        if (mi >= act) break;
        const int ch = 4 * kk + g, r = 16 * mi + c;
        ah[kk][mi] = achunk(as, r, ch);
        al[kk][mi] = achunk(as, BM + r, ch);
      }
    issue_group(kt + QNA - 1);
#pragma unroll
    for (int kk = 0; kk < 2; kk++) {
      bf16x8 b[QFR];
#pragma unroll
      for (int f = 0; f < QFR; f++) {
        const unsigned x = w[f][kk];
        const float y = sc[f][kk];
        const uint4 v = {__builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(x, y, 0)),
                         __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(x, y, 1)),
                         __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(x, y, 2)),
                         __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp4(x, y, 3))};
        b[f] = __builtin_bit_cast(bf16x8, v);
      }
#pragma unroll
      for (int mi = 0; mi < MS; mi++) {
        if (mi >= act) break;
#pragma unroll
        for (int f = 0; f < QFR; f++) {
          acc[mi][f] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[kk][mi], b[f], acc[mi][f], 0, 0, 0);
          acc[mi][f] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[kk][mi], b[f], acc[mi][f], 0, 0, 0);
        }
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(0);  // the clamped tail loads land before the wave ends
  // lane holds C[4 (lane / 16) + i][lane % 16] of each 16 x 16 tile; the
  // slots of its rows are read first (one wait for all of them, not one
  // per row before its stores)
  int slot[MS][4];
#pragma unroll
  for (int mi = 0; mi < MS; mi++)
#pragma unroll
    for (int i = 0; i < 4; i++) slot[mi][i] = p.order[rbeg + min(m0 + 16 * mi + 4 * g + i, cnt - 1)];
#pragma unroll
  for (int mi = 0; mi < MS; mi++)
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int r = 16 * mi + 4 * g + i;
      if (m0 + r >= cnt) continue;
      const int s2 = slot[mi][i];
      if (DUAL && p.y_hi) {  // the down GEMM's A planes, expert order
        const size_t row = (size_t)(rbeg + m0 + r) * p.N;
#pragma unroll
        for (int j = 0; j < HF; j++) {
          const int n = n0 + 16 * HF * wave + 16 * j + c;
          if (n < p.N) {
            const float v = silu_mul(acc[mi][j][i], acc[mi][HF + j][i]);
            const uint16_t h = f32_to_bf16_rne(v);
            p.y_hi[row + n] = h;
            p.y_lo[row + n] = f32_to_bf16_rne(v - bf16_to_f32(h));
          }
        }
      } else if (DUAL) {
#pragma unroll
        for (int j = 0; j < HF; j++) {
          const int n = n0 + 16 * HF * wave + 16 * j + c;
          if (n < p.N) p.y[(size_t)s2 * p.N + n] = silu_mul(acc[mi][j][i], acc[mi][HF + j][i]);
        }
      } else {
#pragma unroll
        for (int f = 0; f < QFR; f++) {
          const int n = n0 + 16 * QFR * wave + 16 * f + c;
          if (n < p.N) p.y[(size_t)s2 * p.N + n] = acc[mi][f][i];
        }
      }
    }
}

// Rows of A in expert order as bf16 hi/lo planes: block i converts the row
// of slot order[i].
__global__ __launch_bounds__(256) void gather_split_kernel(MoeGemmParams p) {
  const int i = blockIdx.x;
  const int slot = p.order[i];
  const float* src = p.a + (size_t)(p.a_per_token ? slot / p.topk : slot) * p.K;
  uint16_t* hi = p.a_hi + (size_t)i * p.K;
  uint16_t* lo = p.a_lo + (size_t)i * p.K;
  for (int k = 4 * threadIdx.x; k < p.K; k += 4 * 256) {
    const float4 x = *(const float4*)(src + k);
    uint16_t h[4], l[4];
    const float v[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
    for (int j = 0; j < 4; j++) {
      h[j] = f32_to_bf16_rne(v[j]);
      l[j] = f32_to_bf16_rne(v[j] - bf16_to_f32(h[j]));
    }
    *(uint2*)(hi + k) = make_uint2(h[0] | ((unsigned)h[1] << 16), h[2] | ((unsigned)h[3] << 16));
    *(uint2*)(lo + k) = make_uint2(l[0] | ((unsigned)l[1] << 16), l[2] | ((unsigned)l[3] << 16));
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
  if (d % 8 || (uintptr_t)router % 16 || (uintptr_t)xn % 16) ST_DIE("MoE router rows must be 16-byte aligned");
  if (d > kRouteDma * kRouteThreads * 4) ST_DIE("MoE router supports embedding_dim <= 8192");
  const size_t shm = (size_t)(d + E) * sizeof(float);
  // STRASGPT_MOE_ROUTE_SCAN=1: the selection for more than 64 experts at
  // any E (for tests: both selections take the same experts)
  const char* sv = getenv("STRASGPT_MOE_ROUTE_SCAN");
  const bool scan = sv && atoi(sv);
  if (E <= WAVE && !scan) {
    set_lds(route_kernel<true>, shm);
    hipLaunchKernelGGL(route_kernel<true>, dim3(T), dim3(kRouteThreads), shm, s, xn, router, E, d, k, sel, sel_w);
  } else {
    set_lds(route_kernel<false>, shm);
    hipLaunchKernelGGL(route_kernel<false>, dim3(T), dim3(kRouteThreads), shm, s, xn, router, E, d, k, sel, sel_w);
  }
  HIP_CHECK(hipGetLastError());
}

bool moe_route_logits_supported(int E, int topk, int d) {
  return E >= 1 && E <= WAVE && topk >= 1 && topk <= E && topk <= 8 && d % 8 == 0 && d >= 8 &&
         d <= kRlXF * 1024 && d <= kRlLd * WAVE * 8;
}

void moe_route_logits(const float* x, const uint16_t* norm_w, float eps, const uint16_t* router, int E, int d,
                      float* logits, float* xn, hipStream_t s) {
  if (!moe_route_logits_supported(E, 1, d)) ST_DIE("decode MoE router shape out of range");
  if (((uintptr_t)router | (uintptr_t)x | (uintptr_t)xn) % 16 || (uintptr_t)norm_w % 8)
    ST_DIE("decode MoE router operands must be aligned");
  const size_t shm = (size_t)d * sizeof(float);
  set_lds(route_logits_kernel, shm);
  hipLaunchKernelGGL(route_logits_kernel, dim3((E + 3) / 4), dim3(256), shm, s, x, norm_w, eps, router, E, d,
                     logits, xn);
  HIP_CHECK(hipGetLastError());
}

void moe_gemv_swiglu(const MoeGemvParams& p, hipStream_t s) {
  if (p.K % 32 || ((uintptr_t)p.blocks | (uintptr_t)p.blocks2) % 16) ST_DIE("MXFP4 rows must be 32-value aligned");
  if (p.topk <= 0 || p.tokens <= 0) ST_DIE("MoE GEMV needs tokens and topk");
  const size_t shm = ((size_t)p.K + 32) * sizeof(float);  // row, then a zero block
  const int rows_per_block = kHalves * kGuRows;
  dim3 grid((p.N + rows_per_block - 1) / rows_per_block, p.tokens * p.topk);
  if (p.K <= 32 * 32 * kSteps && p.K <= kGuDma * kThreads * 4) {
    set_lds(swiglu_kernel<false>, shm);
    hipLaunchKernelGGL(swiglu_kernel<false>, grid, dim3(kThreads), shm, s, p);
  } else {
    set_lds(swiglu_kernel<true>, shm);
    hipLaunchKernelGGL(swiglu_kernel<true>, grid, dim3(kThreads), shm, s, p);
  }
  HIP_CHECK(hipGetLastError());
}

void mxfp4_decode(const uint8_t* codes, const uint8_t* scales, int nblocks, float* out, int bf16_tiles,
                  hipStream_t s) {
  if (nblocks <= 0 || (uintptr_t)codes % 16) ST_DIE("MXFP4 decode needs aligned blocks");
  hipLaunchKernelGGL(mxfp4_decode_kernel, dim3((nblocks + 255) / 256), dim3(256), 0, s, codes, scales,
                     nblocks, out, bf16_tiles);
  HIP_CHECK(hipGetLastError());
}

void moe_gemv_down(const MoeGemvParams& p, hipStream_t s) {
  if (p.K % 32 || (uintptr_t)p.blocks % 16) ST_DIE("MXFP4 rows must be 32-value aligned");
  if (p.topk <= 0 || p.tokens <= 0) ST_DIE("MoE GEMV needs tokens and topk");
  if (p.topk > 8) ST_DIE("MoE down projection supports top-k up to 8");
  const size_t shm = ((size_t)p.topk * p.K + 32) * sizeof(float);
  dim3 grid((p.N + kHalves * kDownRows - 1) / (kHalves * kDownRows), p.tokens);
  const bool loop = p.K > 32 * 32 * kSteps || p.topk * p.K > kDownDma * kThreads * 4;
#define DOWN_CASE(KM, LP)                                                      \
  do {                                                                         \
    set_lds(down_kernel<KM, LP>, shm);                                         \
    hipLaunchKernelGGL((down_kernel<KM, LP>), grid, dim3(kThreads), shm, s, p); \
  } while (0)
  if (p.topk <= 4) {
    if (loop) DOWN_CASE(4, true);
    else DOWN_CASE(4, false);
  } else {
    if (loop) DOWN_CASE(8, true);
    else DOWN_CASE(8, false);
  }
#undef DOWN_CASE
  HIP_CHECK(hipGetLastError());
}

}  // namespace sg

namespace sg {

void moe_group(const int* sel, int n, int E, int* offs, int* order, hipStream_t s) {
  if (n <= 0 || E <= 0 || E > 1024) ST_DIE("MoE grouping needs slots and 1 <= E <= 1024");
  if (E <= WAVE && n <= kGroup2MaxN) {
    static bool attr = false;
    if (!attr) {
      HIP_CHECK(hipFuncSetAttribute((const void*)group2_kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                    (int)(kGroup2MaxN * sizeof(int))));
      attr = true;
    }
    hipLaunchKernelGGL(group2_kernel, dim3(1), dim3(1024), (size_t)n * sizeof(int), s, sel, n, E, offs, order);
  } else {
    hipLaunchKernelGGL(group_kernel, dim3(1), dim3(1024), (E + 1) * sizeof(int), s, sel, n, E, offs, order);
  }
  HIP_CHECK(hipGetLastError());
}

bool moe_group_gemm2_ok(const MoeGemmParams& p) {
  return p.a_hi && p.a_lo && p.K % QKS == 0 && p.K / 32 <= kQMaxNb && p.N % 16 == 0 &&
         !(((uintptr_t)p.blocks | (uintptr_t)p.scales | (uintptr_t)(p.blocks2 ? p.blocks2 : p.blocks) |
            (uintptr_t)(p.scales2 ? p.scales2 : p.scales) | (uintptr_t)p.a_hi | (uintptr_t)p.a_lo) % 16);
}

void moe_gather_split(const MoeGemmParams& p, hipStream_t s) {
  if (!p.a_hi || !p.a_lo || p.K % 4 || (uintptr_t)p.a % 16 || p.slots <= 0) ST_DIE("MoE gather: bad shape");
  hipLaunchKernelGGL(gather_split_kernel, dim3(p.slots), dim3(256), 0, s, p);
  HIP_CHECK(hipGetLastError());
}

// Slots per tile of the grouped GEMM: 64 when the experts average at least
// 24 slots (a 32-slot tiling would stream most experts' weights twice),
// else 32. STRASGPT_MOE_TILE=32|64 forces one (tests run both).
int moe_slot_tile(int slots, int E) {
  const char* v = getenv("STRASGPT_MOE_TILE");
  if (v && *v) {
    const int t = atoi(v);
    if (t != 32 && t != 64) ST_DIE("STRASGPT_MOE_TILE must be 32 or 64");
    return t;
  }
  return slots >= 24 * E ? 64 : 32;
}

void moe_group_gemm(const MoeGemmParams& p, hipStream_t s) {
  if (p.K % 32 || p.N <= 0 || p.slots <= 0) ST_DIE("MoE grouped GEMM shape");
  if ((p.y_hi || p.y_lo) && (!p.y_hi || !p.y_lo || !p.blocks2 || !moe_group_gemm2_ok(p)))
    ST_DIE("MoE grouped GEMM output planes need the pipelined SwiGLU pair");
  if (moe_group_gemm2_ok(p)) {
    const bool dual = p.blocks2 != nullptr;
    const int nb = p.K / 32, runs = dual ? 2 : 1;
    const int bm = moe_slot_tile(p.slots, p.E);
    const size_t shm = (bm == 64 ? QLds<64>::sc : QLds<32>::sc) + (size_t)runs * q_scale_run(QBR / runs, nb);
    const int cols = dual ? QBR / 2 : QBR;
    // slot tiles: an upper bound (the counts are on the device), rounded to
    // whole rounds of the XCDs (the kernel's per-XCD layout)
    const int tmax = ((p.slots + bm - 1) / bm + p.E + kXcds - 1) / kXcds * kXcds;
    const dim3 grid(tmax, (p.N + cols - 1) / cols);
#define GG2(D, B)                                                          \
  do {                                                                     \
    set_lds(group_gemm2_kernel<D, B>, shm);                                \
    hipLaunchKernelGGL((group_gemm2_kernel<D, B>), grid, dim3(256), shm, s, p); \
  } while (0)
    if (dual) {
      if (bm == 64) GG2(true, 64);
      else GG2(true, 32);
    } else {
      if (bm == 64) GG2(false, 64);
      else GG2(false, 32);
    }
#undef GG2
    HIP_CHECK(hipGetLastError());
    return;
  }
  if (((uintptr_t)p.a % 16) || p.K % 4) ST_DIE("MoE grouped GEMM rows must be 16-byte aligned");
  const dim3 grid((p.slots + GBM - 1) / GBM + p.E, (p.N + GBN - 1) / GBN);
  if (p.blocks2)
    hipLaunchKernelGGL(group_gemm_kernel<true>, grid, dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL(group_gemm_kernel<false>, grid, dim3(256), 0, s, p);
  HIP_CHECK(hipGetLastError());
}


}  // namespace sg
