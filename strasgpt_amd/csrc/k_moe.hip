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
constexpr int kDownRows = 2;         // rows per half-wave (down)

// Two values of byte `B` of `w` times `sc` (low nibble first).
template <int B>
__device__ __forceinline__ float2v fp4_pair(uint32_t w, float sc) {
  return __builtin_amdgcn_cvt_scalef32_pk_f32_fp4(w, sc, B);
}

// acc + (block of 32 MXFP4 values, scale sc) . xb[0, 32), in element order.
__device__ __forceinline__ float mx_block_dot(uint4 q, float sc, const float* xb, float acc) {
  const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const float4 xa = *(const float4*)(xb + 8 * i);
    const float4 xc = *(const float4*)(xb + 8 * i + 4);
    const float2v v0 = fp4_pair<0>(w[i], sc), v1 = fp4_pair<1>(w[i], sc);
    const float2v v2 = fp4_pair<2>(w[i], sc), v3 = fp4_pair<3>(w[i], sc);
    acc = fmaf(v0.x, xa.x, acc);
    acc = fmaf(v0.y, xa.y, acc);
    acc = fmaf(v1.x, xa.z, acc);
    acc = fmaf(v1.y, xa.w, acc);
    acc = fmaf(v2.x, xc.x, acc);
    acc = fmaf(v2.y, xc.y, acc);
    acc = fmaf(v3.x, xc.z, acc);
    acc = fmaf(v3.y, xc.w, acc);
  }
  return acc;
}

// Sum over the 32 lanes of a half-wave, the same in each of them.
__device__ __forceinline__ float half_sum(float v) {
#pragma unroll
  for (int off = 16; off >= 1; off >>= 1) v += __shfl_xor(v, off, WAVE);
  return v;
}

// One pass of a half-wave over blocks [b0 + hl, b0 + hl + 32 * kSteps) of
// row `row` (blocks past nb are not loaded): codes and scales into registers.
struct RowLoad {
  uint4 q[kSteps];
  float sc[kSteps];
};

__device__ __forceinline__ void row_load(const uint8_t* blocks, const uint8_t* scales, size_t row,
                                         int nb, int b0, int hl, RowLoad& r) {
  const uint8_t* bq = blocks + row * (size_t)nb * 16;
  const uint8_t* bs = scales + row * (size_t)nb;
#pragma unroll
  for (int i = 0; i < kSteps; i++) {
    const int b = min(b0 + hl + 32 * i, nb - 1);  // past the row: a loaded block, never used
    r.q[i] = load_nt_u4(bq + (size_t)b * 16);
    r.sc[i] = e8m0_scale(bs[b]);
  }
}

__device__ __forceinline__ float row_dot(const RowLoad& r, const float* xs, int nb, int b0, int hl,
                                         float acc) {
#pragma unroll
  for (int i = 0; i < kSteps; i++) {
    const int b = b0 + hl + 32 * i;
    if (b < nb) acc = mx_block_dot(r.q[i], r.sc[i], xs + b * 32, acc);
  }
  return acc;
}

// Router + top-k + softmax, one block of kRouteThreads per token: each
// wave takes experts w, w + 8, ..., kRouteE at a time with every 128-bit
// weight load of those experts in flight before the first is used; wave 0
// then selects.
constexpr int kRouteThreads = 512;
constexpr int kRouteWaves = kRouteThreads / WAVE;
constexpr int kRouteE = 4;     // experts per wave per pass
constexpr int kRouteLd = 6;    // 8-value chunks per lane per expert per pass

__global__ __launch_bounds__(kRouteThreads) void route_kernel(const float* xn, const uint16_t* router,
                                                              int E, int d, int k, int* sel,
                                                              float* sel_w) {
  extern __shared__ __attribute__((aligned(16))) float sm[];
  float* xs = sm;        // [d]
  float* lg = sm + d;    // [E]
  const int t = blockIdx.x, lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  for (int i = threadIdx.x * 4; i < d; i += kRouteThreads * 4)
    *(float4*)(xs + i) = *(const float4*)(xn + (size_t)t * d + i);
  __syncthreads();
  const int chunks = d / 8;
  for (int e0 = wave * kRouteE; e0 < E; e0 += kRouteWaves * kRouteE) {
    float acc[kRouteE];
#pragma unroll
    for (int i = 0; i < kRouteE; i++) acc[i] = 0.0f;
    for (int c0 = 0; c0 < chunks; c0 += kRouteLd * WAVE) {
      uint4 w[kRouteE][kRouteLd];
#pragma unroll
      for (int i = 0; i < kRouteE; i++) {
        const uint16_t* wr = router + (size_t)min(e0 + i, E - 1) * d;
#pragma unroll
        for (int u = 0; u < kRouteLd; u++) w[i][u] = load_nt_u4(wr + min(c0 + u * WAVE + lane, chunks - 1) * 8);
      }
#pragma unroll
      for (int i = 0; i < kRouteE; i++)
#pragma unroll
        for (int u = 0; u < kRouteLd; u++) {
          const int c = c0 + u * WAVE + lane;
          if (c < chunks)
            acc[i] = dot8(w[i][u], *(const float4*)(xs + c * 8), *(const float4*)(xs + c * 8 + 4), acc[i]);
        }
    }
#pragma unroll
    for (int i = 0; i < kRouteE; i++) {
      const float v = wave_sum(acc[i]);
      if (lane == 0 && e0 + i < E) lg[e0 + i] = v;
    }
  }
  __syncthreads();
  if (wave == 0) {
    // k rounds of a wave-wide selection with the semantics of a sequential
    // scan over the experts not yet taken: start from the first, replace
    // on strictly greater (ties keep the lower id; a NaN first candidate
    // stays, later NaNs never win). Lane l holds experts l + 64 m.
    constexpr int kMaxPer = 1024 / WAVE;
    unsigned taken = 0;  // bit m: expert lane + 64 m taken
    int idx[64];
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
      idx[j] = pick;
      if (pick % WAVE == lane) taken |= 1u << (pick / WAVE);
    }
    if (lane == 0) {
      float val[64];
      float sum = 0.0f;
      for (int j = 0; j < k; j++) {
        val[j] = expf(lg[idx[j]] - lg[idx[0]]);
        sum += val[j];
      }
      for (int j = 0; j < k; j++) {
        sel[t * k + j] = idx[j];
        sel_w[t * k + j] = val[j] / sum;
      }
    }
  }
}

// act[s][h] = silu(gate_e[h] . x_s) * (up_e[h] . x_s), slot s = (token, j):
// block (row group, slot); each half-wave takes kGuRows rows of both
// matrices, all their loads of a pass in flight at once.
__global__ __launch_bounds__(kThreads) void swiglu_kernel(MoeGemvParams p) {
  extern __shared__ __attribute__((aligned(16))) float xs[];
  const int slot = blockIdx.y, lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  const int half = wave * 2 + lane / 32, hl = lane % 32;
  const float* xr = p.x + (size_t)(slot / p.topk) * p.K;
  for (int i = threadIdx.x * 4; i < p.K; i += kThreads * 4) *(float4*)(xs + i) = *(const float4*)(xr + i);
  __syncthreads();
  const int e = p.expert[slot];
  const int nb = p.K / 32;
  const int r0 = (blockIdx.x * kHalves + half) * kGuRows;
  float g[kGuRows], u[kGuRows];
#pragma unroll
  for (int r = 0; r < kGuRows; r++) g[r] = u[r] = 0.0f;
  for (int b0 = 0; b0 < nb; b0 += 32 * kSteps) {
    RowLoad lg[kGuRows], lu[kGuRows];
#pragma unroll
    for (int r = 0; r < kGuRows; r++) {
      const size_t row = (size_t)e * p.N + min(r0 + r, p.N - 1);
      row_load(p.blocks, p.scales, row, nb, b0, hl, lg[r]);
      row_load(p.blocks2, p.scales2, row, nb, b0, hl, lu[r]);
    }
#pragma unroll
    for (int r = 0; r < kGuRows; r++) {
      g[r] = row_dot(lg[r], xs, nb, b0, hl, g[r]);
      u[r] = row_dot(lu[r], xs, nb, b0, hl, u[r]);
    }
  }
#pragma unroll
  for (int r = 0; r < kGuRows; r++) {
    const float gs = half_sum(g[r]), us = half_sum(u[r]);
    if (hl == 0 && r0 + r < p.N) p.y[(size_t)slot * p.N + r0 + r] = silu_mul(gs, us);
  }
}

// y[t][n] += sum_j fmaf order of w_j * (down_e_j[n] . act[t*k + j]):
// block (row group, token); each half-wave takes kDownRows rows in turn, for
// every slot of the token, all of a row's loads of a pass in flight at once.
template <int KMAX>
__global__ __launch_bounds__(kThreads) void down_kernel(MoeGemvParams p) {
  extern __shared__ __attribute__((aligned(16))) float as[];  // [k][K]
  const int k = p.topk;
  const int t = blockIdx.y, lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  const int half = wave * 2 + lane / 32, hl = lane % 32;
  for (int i = threadIdx.x * 4; i < k * p.K; i += kThreads * 4)
    *(float4*)(as + i) = *(const float4*)(p.x + (size_t)t * k * p.K + i);
  __syncthreads();
  const int nb = p.K / 32;
  for (int n = (blockIdx.x * kHalves + half) * kDownRows, n1 = n + kDownRows; n < n1; n++) {
    float dot[KMAX];
#pragma unroll
    for (int j = 0; j < KMAX; j++) dot[j] = 0.0f;
    for (int b0 = 0; b0 < nb; b0 += 32 * kSteps) {
      RowLoad ld[KMAX];
#pragma unroll
      for (int j = 0; j < KMAX; j++) {
        const int e = p.expert[t * k + min(j, k - 1)];
        row_load(p.blocks, p.scales, (size_t)e * p.N + min(n, p.N - 1), nb, b0, hl, ld[j]);
      }
#pragma unroll
      for (int j = 0; j < KMAX; j++)
        if (j < k) dot[j] = row_dot(ld[j], as + j * p.K, nb, b0, hl, dot[j]);
    }
    float acc = 0.0f;
#pragma unroll
    for (int j = 0; j < KMAX; j++)
      if (j < k) acc = fmaf(p.weight[t * k + j], half_sum(dot[j]), acc);
    if (hl == 0 && n < p.N) p.y[(size_t)t * p.N + n] += acc;
  }
}

// The decode of mx_block_dot, written out: out[32 b + i] = value i of block b.
__global__ void mxfp4_decode_kernel(const uint8_t* codes, const uint8_t* scales, int nblocks, float* out) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= nblocks) return;
  const uint4 q = *(const uint4*)(codes + (size_t)b * 16);
  const float sc = e8m0_scale(scales[b]);
  const uint32_t w[4] = {q.x, q.y, q.z, q.w};
  float* o = out + (size_t)b * 32;
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

// x[t][n] += sum over j in top-k order of fmaf(w_j, out[t k + j][n], .).
__global__ void combine_kernel(const float* out, const float* w, int T, int k, int N, float* x) {
  const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= (size_t)T * N) return;
  const size_t t = i / N, n = i % N;
  float acc = 0.0f;
  for (int j = 0; j < k; j++) acc = fmaf(w[t * k + j], out[(t * k + j) * N + n], acc);
  x[i] += acc;
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
  const size_t shm = (size_t)(d + E) * sizeof(float);
  set_lds(route_kernel, shm);
  hipLaunchKernelGGL(route_kernel, dim3(T), dim3(kRouteThreads), shm, s, xn, router, E, d, k, sel, sel_w);
  HIP_CHECK(hipGetLastError());
}

void moe_gemv_swiglu(const MoeGemvParams& p, hipStream_t s) {
  if (p.K % 32 || ((uintptr_t)p.blocks | (uintptr_t)p.blocks2) % 16) ST_DIE("MXFP4 rows must be 32-value aligned");
  if (p.topk <= 0 || p.tokens <= 0) ST_DIE("MoE GEMV needs tokens and topk");
  const size_t shm = (size_t)p.K * sizeof(float);
  set_lds(swiglu_kernel, shm);
  const int rows_per_block = kHalves * kGuRows;
  dim3 grid((p.N + rows_per_block - 1) / rows_per_block, p.tokens * p.topk);
  hipLaunchKernelGGL(swiglu_kernel, grid, dim3(kThreads), shm, s, p);
  HIP_CHECK(hipGetLastError());
}

void mxfp4_decode(const uint8_t* codes, const uint8_t* scales, int nblocks, float* out, hipStream_t s) {
  if (nblocks <= 0 || (uintptr_t)codes % 16) ST_DIE("MXFP4 decode needs aligned blocks");
  hipLaunchKernelGGL(mxfp4_decode_kernel, dim3((nblocks + 255) / 256), dim3(256), 0, s, codes, scales,
                     nblocks, out);
  HIP_CHECK(hipGetLastError());
}

void moe_gemv_down(const MoeGemvParams& p, hipStream_t s) {
  if (p.K % 32 || (uintptr_t)p.blocks % 16) ST_DIE("MXFP4 rows must be 32-value aligned");
  if (p.topk <= 0 || p.tokens <= 0) ST_DIE("MoE GEMV needs tokens and topk");
  if (p.topk > 8) ST_DIE("MoE down projection supports top-k up to 8");
  const size_t shm = (size_t)p.topk * p.K * sizeof(float);
  dim3 grid((p.N + kHalves * kDownRows - 1) / (kHalves * kDownRows), p.tokens);
  if (p.topk <= 4) {
    set_lds(down_kernel<4>, shm);
    hipLaunchKernelGGL(down_kernel<4>, grid, dim3(kThreads), shm, s, p);
  } else {
    set_lds(down_kernel<8>, shm);
    hipLaunchKernelGGL(down_kernel<8>, grid, dim3(kThreads), shm, s, p);
  }
  HIP_CHECK(hipGetLastError());
}

}  // namespace sg

namespace sg {

void moe_group(const int* sel, int n, int E, int* offs, int* order, hipStream_t s) {
  if (n <= 0 || E <= 0 || E > 1024) ST_DIE("MoE grouping needs slots and 1 <= E <= 1024");
  hipLaunchKernelGGL(group_kernel, dim3(1), dim3(1024), (E + 1) * sizeof(int), s, sel, n, E, offs, order);
  HIP_CHECK(hipGetLastError());
}

void moe_group_gemm(const MoeGemmParams& p, hipStream_t s) {
  if (p.K % 32 || p.N <= 0 || p.slots <= 0) ST_DIE("MoE grouped GEMM shape");
  if (((uintptr_t)p.a % 16) || p.K % 4) ST_DIE("MoE grouped GEMM rows must be 16-byte aligned");
  const dim3 grid((p.slots + GBM - 1) / GBM + p.E, (p.N + GBN - 1) / GBN);
  if (p.blocks2)
    hipLaunchKernelGGL(group_gemm_kernel<true>, grid, dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL(group_gemm_kernel<false>, grid, dim3(256), 0, s, p);
  HIP_CHECK(hipGetLastError());
}

void moe_combine(const float* out, const float* w, int T, int k, int N, float* x, hipStream_t s) {
  const size_t n = (size_t)T * N;
  hipLaunchKernelGGL(combine_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, out, w, T, k, N, x);
  HIP_CHECK(hipGetLastError());
}

}  // namespace sg
