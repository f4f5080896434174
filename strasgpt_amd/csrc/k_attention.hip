// Causal GQA attention over the device fp32 KV cache
// ([kv_heads][ctx][head_dim] per layer), reference
// source/transformer.c:1375-1422: score = (q . k) / sqrtf(hd), softmax
// with max subtraction and expf, out = sum_s p[s] v[s].
//
// Prefill: fp32 matrix-core flash attention (attn_prefill_mfma_kernel).
//
// Decode: split-K over the cached positions ("flash decoding") in one
// launch: one block per (key chunk, kv head) for all query heads of the
// group writes (max, sum, partial output) per head, and the last block of
// each kv head to finish combines the chunks. The blocks also apply this
// step's QK RMSNorm + RoPE to q and to the new key (read raw from the QKV
// projection); the block holding the newest position writes the processed
// key into the cache.
#include <algorithm>

#include "device_common.h"
#include "hip_check.h"
#include "kernels.h"

namespace sg {

namespace {

typedef __attribute__((address_space(3))) void* lds_ptr;

// Decode: threads per block, keys per LDS tile, query heads per kv head
// and key chunks per kv head, at most.
constexpr int kDecThreads = 256;
constexpr int kDecTile = 32;
constexpr int kDecMaxG = 8;
constexpr int kDecMaxChunks = 64;
constexpr int kDecCombineGroup = 32;  // chunk partials loaded per round of the combine
constexpr int kDecMinChunk = 32;  // keys per chunk, at least

// Split of `total` keys into nch chunks of len keys (the last may be
// shorter, none is empty): as many chunks as allowed, each of at least
// kDecMinChunk keys.
__host__ __device__ inline void attention_decode_split(int total, int max_chunks, int& nch, int& len) {
  nch = total < max_chunks * kDecMinChunk ? (total + kDecMinChunk - 1) / kDecMinChunk : max_chunks;
  len = (total + nch - 1) / nch;
  nch = (total + len - 1) / len;
}

// Prefill attention on the fp32 matrix cores (v_mfma_f32_16x16x4_f32:
// fp32 products accumulated in fp32, as the reference computes them; only
// the summation order differs). Block = 64 queries of one head (4 waves x
// 16 queries), key tiles of 64 brought to LDS by DMA, double-buffered.
// Per tile and wave: S^T = K Q^T (keys as rows: the MFMA output then holds,
// in lane (g, c) = (lane / 16, lane % 16), keys 4g + i of each 16-key
// sub-tile for query c, which is exactly the B operand layout of the P.V
// product's k-steps, so P never leaves registers), the online softmax per
// query (a column: reductions across the four lane groups), then
// O^T += V^T P^T. The head dimension of S^T is walked in an order where a
// lane's four consecutive k-steps read one 16-byte chunk of a K row; K/V
// rows are stored with their 16-byte chunks XOR-swizzled by the row index
// so that the 16 rows read by one instruction hit distinct banks.
constexpr int PQ = 64, PK = 64;

template <int HD>
__device__ __forceinline__ int pre_swz(int row) {
  return row & ((HD / 4 < 16 ? HD / 4 : 16) - 1);
}

// Float offset of (row, d) in a swizzled [PK][HD] tile.
template <int HD>
__device__ __forceinline__ int pre_off(int row, int d) {
  return row * HD + (((d >> 2) ^ pre_swz<HD>(row)) << 2) + (d & 3);
}

// Rows [kv0, kv0 + PK) of a kv head's K and V (clamped to key `last`: the
// rows past it are masked) into swizzled LDS tiles by DMA, 1 KiB per wave
// instruction; lane i of instruction n lands at tile float n*256 + 4i and
// fetches the chunk that belongs there.
template <int HD>
__device__ __forceinline__ void pre_dma(const float* kb, const float* vb, int kv0, int last, float* kt,
                                        float* vt) {
  constexpr int CH = HD / 4, RPK = 256 / HD, NI = PK * HD / 256;
  const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
  for (int n = wave; n < NI; n += 4) {
    const int row = n * RPK + lane / CH, phys = lane % CH;
    const int c = phys ^ pre_swz<HD>(row);
    const size_t key = (size_t)min(kv0 + row, last);
    __builtin_amdgcn_global_load_lds((const void*)(kb + key * HD + c * 4), (lds_ptr)(kt + n * 256), 16, 0, 0);
    __builtin_amdgcn_global_load_lds((const void*)(vb + key * HD + c * 4), (lds_ptr)(vt + n * 256), 16, 0, 0);
  }
}

template <int HD>
__global__ __launch_bounds__(256) void attn_prefill_mfma_kernel(AttnParams p) {
  constexpr int DJ = HD / 16;  // 16-wide slices of the head dimension
  extern __shared__ __attribute__((aligned(16))) float plds[];
  const int lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE, g = lane / 16, c = lane % 16;
  const int nqb = (p.T + PQ - 1) / PQ;
  const int qb = nqb - 1 - (int)blockIdx.x;  // longest causal ranges first
  const int head = blockIdx.y;
  const int G = p.q_heads / p.kv_heads, kvh = head / G;
  const int P = *p.pos, T = p.T;
  const int qd = p.q_heads * HD;
  const int t = qb * PQ + wave * 16 + c;  // this lane's query (column)
  const float* kb = p.kcache + (size_t)kvh * p.ctx * HD;
  const float* vb = p.vcache + (size_t)kvh * p.ctx * HD;
  const int kv_end = P + min(qb * PQ + PQ, T);  // keys visible to the block's last query
  const int ntiles = (kv_end + PK - 1) / PK;
  const float scale = sqrtf((float)HD);

  pre_dma<HD>(kb, vb, 0, kv_end - 1, plds, plds + PK * HD);
  // Q^T operand: lane (g, c) holds q[t][16j + 4g + e] for k-step 4j + e.
  float4 qv[DJ];
  {
    const float* qr = p.q + (size_t)min(t, T - 1) * qd + head * HD + 4 * g;
#pragma unroll
    for (int j = 0; j < DJ; j++) qv[j] = *(const float4*)(qr + 16 * j);
  }
  f32x4 o[DJ];
#pragma unroll
  for (int j = 0; j < DJ; j++) o[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.0f;

  for (int it = 0; it < ntiles; it++) {
    float* kt = plds + (it & 1) * 2 * PK * HD;
    float* vt = kt + PK * HD;
    __builtin_amdgcn_s_waitcnt(0);  // this tile's DMA (and the q loads) landed
    __syncthreads();                // for every wave; the other buffer is free
    if (it + 1 < ntiles) {
      float* nk = plds + ((it + 1) & 1) * 2 * PK * HD;
      pre_dma<HD>(kb, vb, (it + 1) * PK, kv_end - 1, nk, nk + PK * HD);
    }
    const int kv0 = it * PK;
    // S^T[key][query] for the tile's four 16-key sub-tiles.
    f32x4 sc[4];
#pragma unroll
    for (int s4 = 0; s4 < 4; s4++) sc[s4] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < DJ; j++) {
#pragma unroll
      for (int s4 = 0; s4 < 4; s4++) {
        const float4 kv = *(const float4*)(kt + pre_off<HD>(16 * s4 + c, 16 * j + 4 * g));
        sc[s4] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv.x, qv[j].x, sc[s4], 0, 0, 0);
        sc[s4] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv.y, qv[j].y, sc[s4], 0, 0, 0);
        sc[s4] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv.z, qv[j].z, sc[s4], 0, 0, 0);
        sc[s4] = __builtin_amdgcn_mfma_f32_16x16x4f32(kv.w, qv[j].w, sc[s4], 0, 0, 0);
      }
    }
    // Scale, causal mask, online softmax of column t.
    float mx = -INFINITY;
#pragma unroll
    for (int s4 = 0; s4 < 4; s4++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const int key = kv0 + 16 * s4 + 4 * g + i;
        const float v = key <= P + t && key < kv_end ? sc[s4][i] / scale : -INFINITY;
        sc[s4][i] = v;
        mx = fmaxf(mx, v);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16, WAVE));
    mx = fmaxf(mx, __shfl_xor(mx, 32, WAVE));
    const float mn = fmaxf(m, mx);
    const float corr = mn == -INFINITY ? 1.0f : expf(m - mn);
    float rs = 0.0f;
#pragma unroll
    for (int s4 = 0; s4 < 4; s4++)
#pragma unroll
      for (int i = 0; i < 4; i++) {
        const float e = mn == -INFINITY ? 0.0f : expf(sc[s4][i] - mn);
        sc[s4][i] = e;
        rs += e;
      }
    rs += __shfl_xor(rs, 16, WAVE);
    rs += __shfl_xor(rs, 32, WAVE);
    l = l * corr + rs;
    m = mn;
#pragma unroll
    for (int j = 0; j < DJ; j++) o[j] *= corr;
    // O^T[d][query] += V[key][d] P^T[key][query]: k-step (s4, i) covers keys
    // 16 s4 + 4g' + i, g' the lane group, whose P^T values lane (g, c) holds
    // as sc[s4][i].
#pragma unroll
    for (int s4 = 0; s4 < 4; s4++)
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < DJ; j++) {
          const float a = vt[pre_off<HD>(16 * s4 + 4 * g + i, 16 * j + c)];
          o[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, sc[s4][i], o[j], 0, 0, 0);
        }
  }
  // lane (g, c) holds O^T[16j + 4g + e][t]: out[t][head*HD + 16j + 4g + e]
  if (t < T) {
#pragma unroll
    for (int j = 0; j < DJ; j++) {
      const size_t idx = (size_t)t * qd + head * HD + 16 * j + 4 * g;
      uint16_t hi[4], lo[4];
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const float v = o[j][e] / l;
        hi[e] = f32_to_bf16_rne(v);
        lo[e] = f32_to_bf16_rne(v - bf16_to_f32(hi[e]));
      }
      *(uint2*)(p.out_hi + idx) = make_uint2(hi[0] | ((unsigned)hi[1] << 16), hi[2] | ((unsigned)hi[3] << 16));
      if (p.out_lo)
        *(uint2*)(p.out_lo + idx) = make_uint2(lo[0] | ((unsigned)lo[1] << 16), lo[2] | ((unsigned)lo[3] << 16));
    }
  }
}

// LDS layout of the decode kernel (floats).
template <int HD>
struct DecLds {
  static constexpr int KG = kDecThreads / HD;  // key groups for P.V
  static constexpr int qs = 0;                                 // [kDecMaxG][HD]
  static constexpr int kn = qs + kDecMaxG * HD;                // [HD] new key
  static constexpr int sc = kn + HD;                           // [kDecMaxG][kDecTile]
  static constexpr int st = sc + kDecMaxG * kDecTile;          // [3][kDecMaxG] m, l, rescale
  static constexpr int flag = st + 4 * kDecMaxG;               // [4]
  static constexpr int tiles = flag + 4;                       // [2][K|V][kDecTile][HD]
  // After the last tile, over the tile buffers:
  static constexpr int red = tiles;                            // [KG][kDecMaxG][HD]
  static constexpr int wts = red + KG * kDecMaxG * HD;         // [kDecMaxG][kDecMaxChunks + 1]
  static constexpr int total = std::max(tiles + 4 * kDecTile * HD, wts + kDecMaxG * (kDecMaxChunks + 1));
};

// Keys [t0, t0 + n) of a kv head (rows of HD floats, contiguous) into the
// LDS tiles kt / vt by the global-to-LDS DMA: 16 bytes per lane, each wave
// filling 1 KiB of LDS per instruction. No registers are held; the caller
// waits for vector memory operations and syncs the block before reading.
template <int HD>
__device__ __forceinline__ void dma_kv(const float* kb, const float* vb, int t0, int n, float* kt,
                                       float* vt) {
  const int units = n * HD / 4;
  const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
  const float* ks = kb + (size_t)t0 * HD;
  const float* vs = vb + (size_t)t0 * HD;
  for (int u0 = wave * WAVE; u0 < units; u0 += kDecThreads) {
    const int u = u0 + lane;
    if (u < units) {
      __builtin_amdgcn_global_load_lds((const void*)(ks + u * 4), (lds_ptr)(kt + u0 * 4), 16, 0, 0);
      __builtin_amdgcn_global_load_lds((const void*)(vs + u * 4), (lds_ptr)(vt + u0 * 4), 16, 0, 0);
    }
  }
}

// N consecutive floats of LDS into registers, in 16-byte (8-byte for N == 2)
// reads.
template <int N>
__device__ __forceinline__ void lds_read(const float* src, float* dst) {
  if constexpr (N % 4 == 0) {
#pragma unroll
    for (int i = 0; i < N; i += 4) {
      const float4 f = *(const float4*)(src + i);
      dst[i] = f.x;
      dst[i + 1] = f.y;
      dst[i + 2] = f.z;
      dst[i + 3] = f.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < N; i += 2) {
      const float2 f = *(const float2*)(src + i);
      dst[i] = f.x;
      dst[i + 1] = f.y;
    }
  }
}

// RMSNorm (when nw is given) and RoPE of one head vector held by a wave:
// xv / wv are the lane's elements lane + i*64 of the vector and of the norm
// weights, fr / fi the rotation of the lane's pair (element lane*pst and
// lane*pst + po, when lane*pst < pb). Result in LDS dst. Same arithmetic as
// the reference (source/transformer.c:1293-1323).
template <int HD>
__device__ __forceinline__ void norm_rope_regs(const float* xv, const float* wv, bool norm, float eps,
                                               float fr, float fi, int pb, int po, int pst, float* dst) {
#pragma clang fp contract(off)
  constexpr int PER = (HD + WAVE - 1) / WAVE;
  const int lane = threadIdx.x % WAVE;
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < PER; i++)
    if (lane + i * WAVE < HD) ss = fmaf(xv[i], xv[i], ss);
  ss = wave_sum(ss);
  const float s = norm ? rms_scale(ss, HD, eps) : 1.0f;
#pragma unroll
  for (int i = 0; i < PER; i++)
    if (lane + i * WAVE < HD) dst[lane + i * WAVE] = norm ? (xv[i] * s) * wv[i] : xv[i];
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  const int h = lane * pst;
  float r0 = 0.0f, r1 = 0.0f;
  if (h < pb) {
    const float v0 = dst[h], v1 = dst[h + po];
    r0 = v0 * fr - v1 * fi;
    r1 = v0 * fi + v1 * fr;
  }
  __builtin_amdgcn_wave_barrier();
  if (h < pb) {
    dst[h] = r0;
    dst[h + po] = r1;
  }
}

// Decode attention in one launch. Block (chunk c, kv head g) takes keys
// [c*len, min(P+1, (c+1)*len)) for the G query heads of kv head g (the K/V
// rows are read once for the group), in tiles of kDecTile keys brought to
// LDS by DMA, double-buffered: tile t+1 is in flight while tile t is used.
// Per tile: scores (8 lanes per key), an online softmax per head (running
// max m, sum l, rescale of the accumulators), P.V (thread = output dim x
// key group). The block stores (m, l, unnormalised output) per head with
// agent-coherent stores, then counts itself done on the kv head's counter;
// the last block of the head reads all chunks' partials and writes
//   att = sum_c e^(m_c - M) o_c / sum_c e^(m_c - M) l_c,  M = max_c m_c,
// and resets the counter for the next launch. The block holding position
// P also normalises and rotates this step's key and writes it to the
// cache (the value row was written by the QKV projection). Each stage
// issues all its global loads before using any (one memory round trip per
// stage: inputs, partial stores, counter, partial loads).
template <int HD>
__global__ __launch_bounds__(kDecThreads) void attn_decode_kernel(AttnParams p) {
  using L = DecLds<HD>;
  constexpr int KP = HD / 8;  // dims per lane for scores; keys per group for P.V
  constexpr int KG = L::KG;
  constexpr int NW = kDecThreads / WAVE;
  constexpr int PER = (HD + WAVE - 1) / WAVE;
  constexpr int MAXV = (kDecMaxG + 1 + NW - 1) / NW;  // head vectors per wave
  static_assert(kDecTile * 8 == kDecThreads && KG * KP == kDecTile, "tile shape");
  static_assert(kDecMaxChunks <= WAVE, "one lane per chunk in the combine");
  extern __shared__ __attribute__((aligned(16))) float lds[];
  float* qs = lds + L::qs;
  float* kn = lds + L::kn;
  float* sc = lds + L::sc;
  float* st = lds + L::st;
  float* wts = lds + L::wts;
  float* red = lds + L::red;
  int* flag = (int*)(lds + L::flag);
  float* tiles = lds + L::tiles;

  const int c = blockIdx.x, g = blockIdx.y;
  const int G = p.q_heads / p.kv_heads;
  const int P = *p.pos, total = P + 1;
  int nch, len;
  attention_decode_split(total, p.splits, nch, len);
  if (c >= nch) return;  // not counted: the last block waits for nch arrivals
  const int s0 = c * len, s1 = min(total, s0 + len);
  const bool has_new = s1 == total;
  const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
  const float* kb = p.kcache + (size_t)g * p.ctx * HD;
  const float* vb = p.vcache + (size_t)g * p.ctx * HD;

  // Stage 1 loads: the first K/V tile, the raw q (and new k) vectors, their
  // norm weights and the rotation of position P.
  dma_kv<HD>(kb, vb, s0, min(kDecTile, s1 - s0), tiles, tiles + kDecTile * HD);
  const float* cs = p.rope + (size_t)P * HD;
  const int nvec = G + (has_new ? 1 : 0);
  const int hp = lane * p.pair_stride;
  // Loads are unconditional (out-of-range ones read a valid element and are
  // discarded), so that the compiler issues them all before the first use.
  float xv[MAXV][PER], wv[MAXV][PER], fr[MAXV], fi[MAXV];
  const int hq = hp < p.pair_bound ? hp : 0;
#pragma unroll
  for (int j = 0; j < MAXV; j++) {
    const int v = wave + j * NW;
    const bool key = v == G;
    const float* src = key ? p.kraw + (size_t)g * HD : p.q + (size_t)(g * G + (v < G ? v : 0)) * HD;
    const uint16_t* nw = key ? p.kn : p.qn;
    const uint16_t* nws = nw ? nw : (const uint16_t*)src;
#pragma unroll
    for (int i = 0; i < PER; i++) {
      const int e = min(lane + i * WAVE, HD - 1);
      xv[j][i] = src[e];
      wv[j][i] = bf16_to_f32(nws[e]);
    }
    fr[j] = cs[hq];
    fi[j] = cs[hq + p.pair_offset];
  }
#pragma unroll
  for (int j = 0; j < MAXV; j++) {
    const int v = wave + j * NW;
    if (v < nvec)
      norm_rope_regs<HD>(xv[j], wv[j], (v == G ? p.kn : p.qn) != nullptr, p.eps, fr[j], fi[j],
                         p.pair_bound, p.pair_offset, p.pair_stride, v == G ? kn : qs + v * HD);
  }
  if (tid < kDecMaxG) {
    st[tid] = -INFINITY;
    st[kDecMaxG + tid] = 0.0f;
  }
  const float scale = sqrtf((float)HD);
  const int d = tid % HD, kg = tid / HD, kk = tid / 8, pp = tid % 8;
  float acc[kDecMaxG];
#pragma unroll
  for (int h = 0; h < kDecMaxG; h++) acc[h] = 0.0f;

  for (int t0 = s0, buf = 0; t0 < s1; t0 += kDecTile, buf ^= 1) {
    const int n = min(kDecTile, s1 - t0);
    float* kt = tiles + buf * 2 * kDecTile * HD;
    float* vt = kt + kDecTile * HD;
    __builtin_amdgcn_s_waitcnt(0);  // this tile (and the q/k loads) landed
    __syncthreads();                // ... for every wave; previous tile consumed
    if (t0 + kDecTile < s1) {
      float* nk = tiles + (buf ^ 1) * 2 * kDecTile * HD;
      dma_kv<HD>(kb, vb, t0 + kDecTile, min(kDecTile, s1 - t0 - kDecTile), nk, nk + kDecTile * HD);
    }
    if (has_new && P >= t0 && P < t0 + n) {  // row P: this step's processed key
      for (int e = tid; e < HD; e += kDecThreads) kt[(P - t0) * HD + e] = kn[e];
      __syncthreads();
    }
    float kv[KP];
    lds_read<KP>(kt + kk * HD + pp * KP, kv);
#pragma unroll
    for (int h = 0; h < kDecMaxG; h++) {
      if (h < G) {
        float q[KP];
        lds_read<KP>(qs + h * HD + pp * KP, q);
        float a = 0.0f;
#pragma unroll
        for (int i = 0; i < KP; i++) a = fmaf(q[i], kv[i], a);
        a = group_sum<8>(a);
        if (pp == 0) sc[h * kDecTile + kk] = a / scale;
      }
    }
    __syncthreads();
    for (int h = wave; h < G; h += kDecThreads / WAVE) {  // online softmax of head h
      const float s = lane < n ? sc[h * kDecTile + lane] : -INFINITY;
      const float mo = st[h], mn = fmaxf(mo, wave_max(s));
      const float e = lane < n ? expf(s - mn) : 0.0f;
      if (lane < kDecTile) sc[h * kDecTile + lane] = e;  // 0 past the tile's keys
      const float sum = wave_sum(e);
      if (lane == 0) {
        const float f = expf(mo - mn);
        st[2 * kDecMaxG + h] = f;
        st[kDecMaxG + h] = st[kDecMaxG + h] * f + sum;
        st[h] = mn;
      }
    }
    __syncthreads();
    float v[KP];
#pragma unroll
    for (int i = 0; i < KP; i++) v[i] = kg * KP + i < n ? vt[(kg * KP + i) * HD + d] : 0.0f;
#pragma unroll
    for (int h = 0; h < kDecMaxG; h++) {
      if (h < G) {
        float w[KP];
        lds_read<KP>(sc + h * kDecTile + kg * KP, w);
        float a = acc[h] * st[2 * kDecMaxG + h];
#pragma unroll
        for (int i = 0; i < KP; i++) a = fmaf(w[i], v[i], a);
        acc[h] = a;
      }
    }
  }
  __syncthreads();  // last tile consumed (red overlaps the tiles)
#pragma unroll
  for (int h = 0; h < kDecMaxG; h++)
    if (h < G) red[(kg * kDecMaxG + h) * HD + d] = acc[h];
  __syncthreads();
  for (int o = tid; o < G * HD; o += kDecThreads) {
    const int h = o / HD, dd = o % HD;
    float a = 0.0f;
#pragma unroll
    for (int k = 0; k < KG; k++) a += red[(k * kDecMaxG + h) * HD + dd];
    float* part = p.partial + ((size_t)(g * G + h) * p.splits + c) * (HD + 2);
    cstore(part + 2 + dd, a);
    if (dd == 0) {
      cstore(part, st[h]);
      cstore(part + 1, st[kDecMaxG + h]);
    }
  }
  if (has_new) {  // cache row P of kv head g, read by later steps
    float* kc = p.kcache_w + ((size_t)g * p.ctx + P) * HD;
    for (int e = tid; e < HD; e += kDecThreads) kc[e] = kn[e];
  }
  __builtin_amdgcn_s_waitcnt(0);  // partials stored (agent-coherent)
  __syncthreads();
  if (tid == 0) {
    const unsigned done = __hip_atomic_fetch_add(p.counters + g, 1u, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
    flag[0] = done == (unsigned)(nch - 1);
  }
  __syncthreads();
  if (!flag[0]) return;

  // Last block of kv head g: combine the nch chunks of its G heads, two
  // outputs per thread at a time (one round for G * HD <= 512), the chunk
  // partials in groups of 32 loaded before any is used.
  float m[MAXV], l[MAXV];
#pragma unroll
  for (int j = 0; j < MAXV; j++) {
    const int h = wave + j * NW;
    const float* pb = p.partial + (size_t)(g * G + h) * p.splits * (HD + 2) + (size_t)lane * (HD + 2);
    const bool ok = h < G && lane < nch;
    m[j] = ok ? cload(pb) : -INFINITY;
    l[j] = ok ? cload(pb + 1) : 0.0f;
  }
  constexpr int CG = kDecCombineGroup;
  for (int o0 = 0; o0 < G * HD; o0 += 2 * kDecThreads) {
    float a[2] = {0.0f, 0.0f};
    for (int c0 = 0; c0 < nch; c0 += CG) {
      float x[2][CG];
#pragma unroll
      for (int r = 0; r < 2; r++) {
        const int o = min(o0 + tid + r * kDecThreads, G * HD - 1), h = o / HD, dd = o % HD;
        const float* pb = p.partial + (size_t)(g * G + h) * p.splits * (HD + 2) + 2 + dd;
#pragma unroll
        for (int i = 0; i < CG; i++) x[r][i] = cload(pb + (size_t)min(c0 + i, nch - 1) * (HD + 2));
      }
      if (o0 == 0 && c0 == 0) {
#pragma unroll
        for (int j = 0; j < MAXV; j++) {
          const int h = wave + j * NW;
          if (h < G) {
            const float M = wave_max(m[j]);
            const float w = lane < nch ? expf(m[j] - M) : 0.0f;
            if (lane < kDecMaxChunks) wts[h * (kDecMaxChunks + 1) + lane] = w;
            const float wl = wave_sum(w * l[j]);
            if (lane == 0) wts[h * (kDecMaxChunks + 1) + kDecMaxChunks] = wl;
          }
        }
        __syncthreads();
      }
#pragma unroll
      for (int r = 0; r < 2; r++) {
        const int h = min(o0 + tid + r * kDecThreads, G * HD - 1) / HD;
        const float* w = wts + h * (kDecMaxChunks + 1) + c0;
#pragma unroll
        for (int i = 0; i < CG; i++)
          if (c0 + i < nch) a[r] = fmaf(w[i], x[r][i], a[r]);
      }
    }
#pragma unroll
    for (int r = 0; r < 2; r++) {
      const int o = o0 + tid + r * kDecThreads, h = o / HD, dd = o % HD;
      if (o < G * HD) p.out[(size_t)(g * G + h) * HD + dd] = a[r] / wts[h * (kDecMaxChunks + 1) + kDecMaxChunks];
    }
  }
  if (tid == 0) __hip_atomic_store(p.counters + g, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

// Chunks per kv head: up to 512 blocks (two per CU fit at once).
int attention_decode_chunks(int kv_heads) {
  return std::max(1, std::min(kDecMaxChunks, 512 / std::max(1, kv_heads)));
}

void attention_init() {
  HIP_CHECK(hipFuncSetAttribute((const void*)attn_prefill_mfma_kernel<16>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, 4 * PK * 16 * (int)sizeof(float)));
  HIP_CHECK(hipFuncSetAttribute((const void*)attn_prefill_mfma_kernel<32>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, 4 * PK * 32 * (int)sizeof(float)));
  HIP_CHECK(hipFuncSetAttribute((const void*)attn_prefill_mfma_kernel<64>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, 4 * PK * 64 * (int)sizeof(float)));
  HIP_CHECK(hipFuncSetAttribute((const void*)attn_prefill_mfma_kernel<128>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, 4 * PK * 128 * (int)sizeof(float)));
  HIP_CHECK(hipFuncSetAttribute((const void*)attn_decode_kernel<16>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)(DecLds<16>::total * sizeof(float))));
  HIP_CHECK(hipFuncSetAttribute((const void*)attn_decode_kernel<32>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)(DecLds<32>::total * sizeof(float))));
  HIP_CHECK(hipFuncSetAttribute((const void*)attn_decode_kernel<64>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)(DecLds<64>::total * sizeof(float))));
  HIP_CHECK(hipFuncSetAttribute((const void*)attn_decode_kernel<128>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)(DecLds<128>::total * sizeof(float))));
}

size_t attention_decode_lds_bytes(int hd) {
  switch (hd) {
    case 16: return DecLds<16>::total * sizeof(float);
    case 32: return DecLds<32>::total * sizeof(float);
    case 64: return DecLds<64>::total * sizeof(float);
    case 128: return DecLds<128>::total * sizeof(float);
    default: return 0;
  }
}

void attention_prefill(const AttnParams& p, hipStream_t s) {
  if (p.T <= 0 || p.q_heads % p.kv_heads) ST_DIE("bad attention shape");
  if (!p.out_hi) ST_DIE("prefill attention writes bf16 planes");
  dim3 grid((p.T + PQ - 1) / PQ, p.q_heads);
  switch (p.hd) {
#define PREFILL_CASE(HD)                                                                         \
  case HD:                                                                                       \
    hipLaunchKernelGGL(attn_prefill_mfma_kernel<HD>, grid, dim3(256), 4 * PK * HD * sizeof(float), s, p); \
    break;
    PREFILL_CASE(16)
    PREFILL_CASE(32)
    PREFILL_CASE(64)
    PREFILL_CASE(128)
#undef PREFILL_CASE
    default: ST_DIE("attention supports head_dim 16, 32, 64 or 128");
  }
  HIP_CHECK(hipGetLastError());
}

void attention_decode(const AttnParams& p, hipStream_t s) {
  const int G = p.kv_heads > 0 ? p.q_heads / p.kv_heads : 0;
  if (G <= 0 || p.q_heads % p.kv_heads) ST_DIE("bad attention shape");
  if (G > kDecMaxG) ST_DIE("decode attention supports at most 8 query heads per kv head");
  if (p.splits < 1 || p.splits > kDecMaxChunks) ST_DIE("decode attention chunk count out of range");
  if (!p.counters || !p.partial) ST_DIE("decode attention needs its partial buffer and counters");
  if (p.pair_stride < 1 || (p.pair_bound + p.pair_stride - 1) / p.pair_stride > WAVE ||
      p.pair_bound - p.pair_stride + p.pair_offset >= p.hd)
    ST_DIE("decode attention: RoPE pairs must fit one per lane within the head");
  const dim3 grid(p.splits, p.kv_heads);
  const size_t shm = attention_decode_lds_bytes(p.hd);
  switch (p.hd) {
#define DECODE_CASE(HD)                                                              \
  case HD:                                                                           \
    hipLaunchKernelGGL(attn_decode_kernel<HD>, grid, dim3(kDecThreads), shm, s, p); \
    break;
    DECODE_CASE(16)
    DECODE_CASE(32)
    DECODE_CASE(64)
    DECODE_CASE(128)
#undef DECODE_CASE
    default: ST_DIE("attention supports head_dim 16, 32, 64 or 128");
  }
  HIP_CHECK(hipGetLastError());
}

}  // namespace sg
