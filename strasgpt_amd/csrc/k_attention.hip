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
#include <cstdlib>
#include <cstring>

#include "device_common.h"
#include "hip_check.h"
#include "kernels.h"

namespace sg {

namespace {

typedef __attribute__((address_space(3))) void* lds_ptr;

// Decode: threads per block, query heads per kv head and blocks (partial
// results) per kv head, at most.
constexpr int kDecMaxG = 8;
constexpr int kDecMaxChunks = 64;

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
constexpr int kX3Keys = 32;  // key tile of the split-bf16 kernel

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
template <int HD, int ROWS = PK>
__device__ __forceinline__ void pre_dma(const float* kb, const float* vb, int kv0, int last, float* kt,
                                        float* vt) {
  constexpr int CH = HD / 4, RPK = 256 / HD, NI = ROWS * HD / 256;
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
  const int P = *p.pos + p.q0, T = p.T;
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
      if (!p.out_hi) {  // fp32 rows (the multi-row GEMV's input)
        *(float4*)(p.out + idx) = make_float4(o[j][0] / l, o[j][1] / l, o[j][2] / l, o[j][3] / l);
        continue;
      }
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

// Prefill attention on the bf16 matrix cores with split operands
// (v_mfma_f32_16x16x32_bf16). Every fp32 operand x is split into
// hi = bf16(x) and lo = bf16(x - hi) (x - hi is exact in fp32), and each
// product is formed as hi*hi' + hi*lo' + lo*hi' in the fp32 accumulator:
// the dropped lo*lo' term and the remainders of the split are below
// 2^-16 of the product, against the 2^-24 of an fp32 product, at 3 bf16
// MFMAs (16 cycles each for 16x16x32) where the fp32 matrix cores take 32
// cycles per 16x16x4. The causal structure, the online softmax and the
// summation per query follow the fp32 kernel above.
//
// Block = 64 queries of one head (4 waves x 16), key tiles of 32. Each
// thread loads its share of the next tile's fp32 K and V rows into
// registers while the current tile is multiplied, splits them once for the
// whole block and stores bf16 hi/lo planes to LDS: K as rows [key][HD]
// (16-byte chunks XOR-swizzled by key), V transposed [HD][32 keys] (chunks
// swizzled by d), double-buffered (64 KiB at head_dim 128: two blocks per
// CU). Per tile and wave:
// * S^T = K Q^T: A operand row c of key sub-tile s is key
//   8 (c / 4) + 4 s + c % 4, so that the output lane (g, c) holds keys
//   8 g .. 8 g + 7 of query c; B operand = the query's split values, kept
//   in registers for the whole block.
// * O^T += V^T P^T over the tile's 32 keys as one MFMA k-step: P^T is the
//   B operand straight from the scores a lane holds; the A operand is one
//   16-byte read of V^T (row 16 dj + c, keys 8 g ..) per plane.
// head_dim 16 pads the 32-dim k-step of S with zeros (lanes g >= 2).
// Lane l's value plus / max with lane l ^ 16 or l ^ 32 (gfx950 lane-swap
// moves: no LDS round trip), and lane l ^ 8 within a row of 16 (DPP).
__device__ __forceinline__ float xor16_sum(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor32_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float xor16_max(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xor32_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float dpp_ror8(float x) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x128, 0xf, 0xf, false));  // row_ror:8
}


template <int HD>
struct X3Lds {
  static constexpr int KP = kX3Keys * HD;  // bf16 elements per K plane
  static constexpr int VP = HD * kX3Keys;  // per V^T plane
  static constexpr int buf = 2 * KP + 2 * VP;  // one tile: K hi, K lo, V^T hi, V^T lo
  static constexpr int bytes = 2 * buf * 2;    // two buffers of bf16
};

template <int HD>
__device__ __forceinline__ int x3_kswz(int key) {
  constexpr int CH = HD / 8;  // 16-byte chunks per K row
  return CH >= 4 ? (key ^ (key >> 2)) & (CH - 1) : (key >> 2) & (CH - 1);
}
__device__ __forceinline__ int x3_vswz(int d) { return (0 - (d >> 2)) & 3; }

// Cache rows [r0, r1) of one kv head (blockIdx.y) into the bf16 planes:
// 32 rows per block. K keeps its row layout; V goes through LDS and is
// written transposed, 64 contiguous bytes (32 keys) per dim and plane.
// A bf16 cache (B16) holds rows that are bf16 already: their split is the
// row itself and a zero lo plane.
template <int HD, bool B16>
__device__ __forceinline__ float2 cache_pair(const float* c, size_t i) {
  if constexpr (B16) {
    const uint32_t u = *(const uint32_t*)((const uint16_t*)c + i);
    return make_float2(__uint_as_float(u << 16), __uint_as_float(u & 0xFFFF0000u));
  } else {
    return *(const float2*)(c + i);
  }
}
template <bool B16>
__device__ __forceinline__ float cache_at(const float* c, size_t i) {
  if constexpr (B16) return bf16_to_f32(((const uint16_t*)c)[i]);
  else return c[i];
}

template <int HD, bool B16>
__global__ __launch_bounds__(256) void split_rows_kernel(const float* kc, const float* vc, uint16_t* khi,
                                                         uint16_t* klo, uint16_t* vthi, uint16_t* vtlo,
                                                         int ctx, int ctx_pad, int r0, int r1) {
  // every load of the thread is issued before the first is used (a loop of
  // load, convert, store per element waits a memory latency per element)
  constexpr int KP = 32 * HD / 2 / 256;  // K pairs per thread
  constexpr int VE = 32 * HD / 256;      // V elements per thread
  __shared__ float vs[32][HD + 1];
  const int tid = threadIdx.x, h = blockIdx.y;
  const int rb = r0 + blockIdx.x * 32;  // first row of the block
  const size_t kbase = (size_t)h * ctx * HD;
  float2 kx[KP];
  float vx[VE];
#pragma unroll
  for (int j = 0; j < KP; j++) {
    const int i = tid + 256 * j, r = min(rb + (2 * i) / HD, r1 - 1), dd = (2 * i) % HD;
    kx[j] = cache_pair<HD, B16>(kc, kbase + (size_t)r * HD + dd);
  }
#pragma unroll
  for (int j = 0; j < VE; j++) {
    const int i = tid + 256 * j, r = min(rb + i / HD, r1 - 1), dd = i % HD;
    vx[j] = cache_at<B16>(vc, kbase + (size_t)r * HD + dd);
  }
#pragma unroll
  for (int j = 0; j < KP; j++) {
    const int i = tid + 256 * j, r = rb + (2 * i) / HD, dd = (2 * i) % HD;
    if (r < r1) {
      uint32_t hi, lo;
      split2(kx[j].x, kx[j].y, hi, lo);
      *(uint32_t*)(khi + kbase + (size_t)r * HD + dd) = hi;
      *(uint32_t*)(klo + kbase + (size_t)r * HD + dd) = lo;
    }
  }
#pragma unroll
  for (int j = 0; j < VE; j++) {
    const int i = tid + 256 * j;
    vs[i / HD][i % HD] = rb + i / HD < r1 ? vx[j] : 0.0f;
  }
  __syncthreads();
  const size_t vbase = (size_t)h * HD * ctx_pad;
  for (int i = tid; i < HD * 16; i += 256) {
    const int dd = i / 16, k2 = 2 * (i % 16);  // keys rb + k2, + 1
    if (rb + k2 < r1) {  // r1 is even or the odd last key's partner is beyond r1 (zero)
      uint32_t hi, lo;
      split2(vs[k2][dd], vs[k2 + 1][dd], hi, lo);
      if (rb + k2 + 1 >= r1) {  // keep the partner's stored value (not yet converted)
        hi &= 0xFFFFu;
        lo &= 0xFFFFu;
        const size_t o = vbase + (size_t)dd * ctx_pad + rb + k2;
        vthi[o] = (uint16_t)hi;
        vtlo[o] = (uint16_t)lo;
      } else {
        *(uint32_t*)(vthi + vbase + (size_t)dd * ctx_pad + rb + k2) = hi;
        *(uint32_t*)(vtlo + vbase + (size_t)dd * ctx_pad + rb + k2) = lo;
      }
    }
  }
}

// QS query sub-tiles of 16 per wave (PQ = 64 QS queries per block): the K
// and V fragments a wave reads from LDS for a tile serve all of them, so
// QS = 2 halves the LDS reads per product (the kernel is bound by them).
template <int HD, int QS>
__global__ __launch_bounds__(256, 2) void attn_prefill_x3_kernel(AttnParams p) {
  constexpr int KT = kX3Keys;              // keys per tile
  constexpr int NKK = (HD + 31) / 32;      // 32-dim k-steps of S
  constexpr int DJ = HD / 16;              // 16-dim sub-tiles of O
  constexpr int PQB = PQ * QS;             // queries per block
  using L = X3Lds<HD>;
  static_assert(L::KP % 512 == 0 && L::VP % 512 == 0, "planes split into 1 KiB DMA instructions");
  constexpr int NKI = L::KP / 512, NVI = L::VP / 512;  // 1 KiB instructions per plane
  extern __shared__ __attribute__((aligned(16))) uint16_t xl[];
  const int lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE, g = lane / 16, c = lane % 16;
  const int nqb = (p.T + PQB - 1) / PQB;
  // grid (heads, query blocks): blocks are dispatched head-fastest, so
  // every head's longest causal range goes first and the shortest last
  const int qb = nqb - 1 - (int)blockIdx.y;
  const int head = blockIdx.x;
  const int G = p.q_heads / p.kv_heads, kvh = head / G;
  const int P = *p.pos + p.q0, T = p.T;
  const int qd = p.q_heads * HD;
  int t[QS];  // this lane's queries
#pragma unroll
  for (int q = 0; q < QS; q++) t[q] = qb * PQB + wave * 16 * QS + 16 * q + c;
  const uint16_t* khg = p.khi + (size_t)kvh * p.ctx * HD;
  const uint16_t* klg = p.klo + (size_t)kvh * p.ctx * HD;
  const uint16_t* vhg = p.vthi + (size_t)kvh * HD * p.ctx_pad;
  const uint16_t* vlg = p.vtlo + (size_t)kvh * HD * p.ctx_pad;
  const int kv_end = P + min(qb * PQB + PQB, T);  // keys visible to the block's last query
  const int ntiles = (kv_end + KT - 1) / KT;
  // scores in the base-2 domain: s * log2(e) / sqrt(HD)
  const float sl2 = 1.44269504088896341f / sqrtf((float)HD);
  // last key visible to each of this lane's queries, and to every query of the block
  int vis[QS];
#pragma unroll
  for (int q = 0; q < QS; q++) vis[q] = min(P + t[q], kv_end - 1);
  const int vis_all = min(P + qb * PQB, kv_end - 1);

  auto split8 = [](const float (&x)[8], bf16x8& hi, bf16x8& lo) {
    uint32_t h[4], l[4];
#pragma unroll
    for (int e = 0; e < 4; e++) split2(x[2 * e], x[2 * e + 1], h[e], l[e]);
    hi = __builtin_bit_cast(bf16x8, (uint4){h[0], h[1], h[2], h[3]});
    lo = __builtin_bit_cast(bf16x8, (uint4){l[0], l[1], l[2], l[3]});
  };
  // One tile's planes into LDS buffer buf by the global-to-LDS DMA: lane i
  // of instruction n lands at plane element 512 n + 8 i and fetches the
  // logical chunk that belongs there. K rows past the last visible key load
  // that key (masked later); V^T rows cover keys kv0 .. kv0 + 31 < ctx_pad
  // (entries never converted are zero, finite).
  auto dma_tile = [&](int kv0, uint16_t* buf) {
    for (int n = wave; n < NKI; n += 4) {
      const int e = 512 * n + 8 * lane, row = e / HD, phys = (e % HD) / 8;
      const int lc = phys ^ x3_kswz<HD>(row);
      const size_t src = (size_t)min(kv0 + row, kv_end - 1) * HD + 8 * lc;
      __builtin_amdgcn_global_load_lds((const void*)(khg + src), (lds_ptr)(buf + 512 * n), 16, 0, 0);
      __builtin_amdgcn_global_load_lds((const void*)(klg + src), (lds_ptr)(buf + L::KP + 512 * n), 16, 0, 0);
    }
    for (int n = wave; n < NVI; n += 4) {
      const int e = 512 * n + 8 * lane, d = e / KT, phys = (e % KT) / 8;
      const int lc = phys ^ x3_vswz(d);
      const size_t src = (size_t)d * p.ctx_pad + kv0 + 8 * lc;
      __builtin_amdgcn_global_load_lds((const void*)(vhg + src), (lds_ptr)(buf + 2 * L::KP + 512 * n), 16, 0,
                                       0);
      __builtin_amdgcn_global_load_lds((const void*)(vlg + src),
                                       (lds_ptr)(buf + 2 * L::KP + L::VP + 512 * n), 16, 0, 0);
    }
  };

  dma_tile(0, xl);
  // Q^T operands: lane (g, c) holds q[t][32 kk + 8 g .. + 7], split.
  bf16x8 qh[QS][NKK], ql[QS][NKK];
#pragma unroll
  for (int q = 0; q < QS; q++) {
    const float* qr = p.q + (size_t)min(t[q], T - 1) * qd + head * HD;
#pragma unroll
    for (int kk = 0; kk < NKK; kk++) {
      float x[8];
      const int d = 32 * kk + 8 * g;
      if (d < HD) {  // the base-2 score scale folded into q
        const float4 a = *(const float4*)(qr + d), b = *(const float4*)(qr + d + 4);
        x[0] = a.x * sl2; x[1] = a.y * sl2; x[2] = a.z * sl2; x[3] = a.w * sl2;
        x[4] = b.x * sl2; x[5] = b.y * sl2; x[6] = b.z * sl2; x[7] = b.w * sl2;
      } else {
#pragma unroll
        for (int e = 0; e < 8; e++) x[e] = 0.0f;
      }
      split8(x, qh[q][kk], ql[q][kk]);
    }
  }

  f32x4 o[QS][DJ];
  float m[QS], l[QS];
#pragma unroll
  for (int q = 0; q < QS; q++) {
#pragma unroll
    for (int j = 0; j < DJ; j++) o[q][j] = f32x4{0.f, 0.f, 0.f, 0.f};
    m[q] = -INFINITY;
    l[q] = 0.0f;
  }
  // Per-lane parts of the LDS addresses (elements).
  int krow[2], kx[2];
#pragma unroll
  for (int s = 0; s < 2; s++) {
    const int key = 8 * (c >> 2) + 4 * s + (c & 3);
    krow[s] = key * HD;
    kx[s] = x3_kswz<HD>(key);
  }
  const int vrow = c * KT + ((g ^ x3_vswz(c)) << 3);  // + 16 dj * KT

  for (int it = 0; it < ntiles; it++) {
    __builtin_amdgcn_s_waitcnt(0);  // this tile's DMA (and the q loads) landed
    __syncthreads();                // for every wave; the other buffer is free
    if (it + 1 < ntiles) dma_tile((it + 1) * KT, xl + ((it + 1) & 1) * L::buf);
    const uint16_t* buf = xl + (it & 1) * L::buf;
    const uint16_t* khi = buf;
    const uint16_t* klo = buf + L::KP;
    const uint16_t* vhi = buf + 2 * L::KP;
    const uint16_t* vlo = vhi + L::VP;
    const int kv0 = it * KT;
    f32x4 sc[QS][2];
#pragma unroll
    for (int s = 0; s < 2; s++) {
#pragma unroll
      for (int q = 0; q < QS; q++) sc[q][s] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < NKK; kk++) {
        // dims past HD (head_dim 16: lane groups 2, 3) are zero in both
        // operands; the MFMAs run on the whole wavefront
        bf16x8 kh = {}, kl = {};
        if (32 * kk + 8 * g < HD) {
          const int off = krow[s] + (((4 * kk + g) ^ kx[s]) << 3);
          kh = *(const bf16x8*)(khi + off);
          kl = *(const bf16x8*)(klo + off);
        }
#pragma unroll
        for (int q = 0; q < QS; q++) {
          sc[q][s] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kh, qh[q][kk], sc[q][s], 0, 0, 0);
          sc[q][s] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kh, ql[q][kk], sc[q][s], 0, 0, 0);
          sc[q][s] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kl, qh[q][kk], sc[q][s], 0, 0, 0);
        }
      }
    }
    // Causal mask and online softmax of each query (base 2; lane groups g
    // hold keys 8 g .. 8 g + 7 of the tile). The reference point m moves
    // only when a query's tile maximum exceeds it by more than 8 (p then
    // stays below 2^8), and then for the whole wave at once: most tiles
    // skip the rescale of O and l. Key 0 is visible to every query, so m is
    // finite from the first tile on and a fully masked row gives p = 0.
    bf16x8 ph[QS], pl[QS];
    const bool full = kv0 + KT - 1 <= vis_all;  // every key of the tile visible to every query of the block
#pragma unroll
    for (int q = 0; q < QS; q++) {
      float pv[8];
      if (full) {
#pragma unroll
        for (int j = 0; j < 8; j++) pv[j] = sc[q][j >> 2][j & 3];
      } else {
#pragma unroll
        for (int j = 0; j < 8; j++) pv[j] = kv0 + 8 * g + j <= vis[q] ? sc[q][j >> 2][j & 3] : -INFINITY;
      }
      float mx = fmaxf(fmaxf(fmaxf(pv[0], pv[1]), fmaxf(pv[2], pv[3])), fmaxf(fmaxf(pv[4], pv[5]), fmaxf(pv[6], pv[7])));
      mx = fmaxf(mx, xor16_max(mx));
      mx = fmaxf(mx, xor32_max(mx));
      const bool up = mx > m[q] + 8.0f;  // (m = -inf before the first tile)
      if (__builtin_amdgcn_ballot_w64(up)) {
        const float mn = up ? mx : m[q];
        const float corr = __builtin_amdgcn_exp2f(m[q] - mn);  // 0 at the first tile (o, l are 0)
        l[q] *= corr;
#pragma unroll
        for (int j = 0; j < DJ; j++) o[q][j] *= corr;
        m[q] = mn;
      }
      float rs = 0.0f;
#pragma unroll
      for (int j = 0; j < 8; j++) {
        const float e = __builtin_amdgcn_exp2f(pv[j] - m[q]);
        pv[j] = e;
        rs += e;
      }
      rs = xor16_sum(rs);
      rs = xor32_sum(rs);
      l[q] += rs;
      split8(pv, ph[q], pl[q]);
    }
#pragma unroll
    for (int dj = 0; dj < DJ; dj++) {
      const bf16x8 vh = *(const bf16x8*)(vhi + vrow + 16 * dj * KT);
      const bf16x8 vl = *(const bf16x8*)(vlo + vrow + 16 * dj * KT);
#pragma unroll
      for (int q = 0; q < QS; q++) {
        o[q][dj] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vh, ph[q], o[q][dj], 0, 0, 0);
        o[q][dj] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vh, pl[q], o[q][dj], 0, 0, 0);
        o[q][dj] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vl, ph[q], o[q][dj], 0, 0, 0);
      }
    }
  }
  // lane (g, c) holds O^T[16 dj + 4 g + e][t]: out[t][head*HD + 16 dj + 4 g + e]
#pragma unroll
  for (int q = 0; q < QS; q++) {
    if (t[q] >= T) continue;
#pragma unroll
    for (int j = 0; j < DJ; j++) {
      const size_t idx = (size_t)t[q] * qd + head * HD + 16 * j + 4 * g;
      if (!p.out_hi) {  // fp32 rows (the multi-row GEMV's input)
        *(float4*)(p.out + idx) = make_float4(o[q][j][0] / l[q], o[q][j][1] / l[q], o[q][j][2] / l[q],
                                              o[q][j][3] / l[q]);
        continue;
      }
      uint16_t hi[4], lo[4];
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const float v = o[q][j][e] / l[q];
        hi[e] = f32_to_bf16_rne(v);
        lo[e] = f32_to_bf16_rne(v - bf16_to_f32(hi[e]));
      }
      *(uint2*)(p.out_hi + idx) = make_uint2(hi[0] | ((unsigned)hi[1] << 16), hi[2] | ((unsigned)hi[3] << 16));
      if (p.out_lo)
        *(uint2*)(p.out_lo + idx) = make_uint2(lo[0] | ((unsigned)lo[1] << 16), lo[2] | ((unsigned)lo[3] << 16));
    }
  }
}

// RMSNorm (when nw is given) and RoPE of one head vector held by a wave:
// xv / wv are the lane's elements lane + i*64 of the vector and of the norm
// weights, fr / fi the rotation of the lane's pair (element lane*pst and
// lane*pst + po, when lane*pst < pb). Result in LDS dst. Same arithmetic as
// the reference (source/transformer.c:1293-1323).
__device__ __forceinline__ float round_bf16(float x) { return bf16_to_f32(f32_to_bf16_any(x)); }

// B16: the result is rounded to bf16 (a key headed for a bf16 cache).
template <int HD, bool B16 = false>
__device__ __forceinline__ void norm_rope_regs(const float* xv, const float* wv, bool norm, float eps,
                                               float fr, float fi, int pb, int po, int pst, float* dst) {
#pragma clang fp contract(off)
  constexpr int PER = (HD + WAVE - 1) / WAVE;
  const int lane = threadIdx.x % WAVE;
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < PER; i++)
    if (lane + i * WAVE < HD) ss = fmaf(xv[i], xv[i], ss);
  ss = wave_total(ss);
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
    dst[h] = B16 ? round_bf16(r0) : r0;
    dst[h + po] = B16 ? round_bf16(r1) : r1;
  }
  if constexpr (B16) {  // elements outside every rotated pair, rounded too
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int i = 0; i < PER; i++) {
      const int e = lane + i * WAVE;
      const bool first = e < pb && e % pst == 0, second = e >= po && e - po < pb && (e - po) % pst == 0;
      if (e < HD && !first && !second) dst[e] = round_bf16(dst[e]);
    }
  }
}


// Decode attention on the matrix cores, over the cache's bf16 planes (the
// operands of the split-bf16 prefill kernel: K [kv][ctx][hd] hi/lo, V
// transposed [kv][hd][ctx_pad] hi/lo; with a bf16 cache the hi planes hold
// the rows and lo is not read).
//
// Block (b, kv head g) takes tiles [b*tpb, (b+1)*tpb) of 32 keys; wave w
// takes tiles w, w+4, ... of them (waves without a tile only help with the
// queries), their operands loaded straight into registers in the MFMA
// layouts (no LDS), with its own online softmax state for all G query
// heads at once:
// * S^T = K Q^T by v_mfma_f32_16x16x32_bf16: the query heads are the 16
//   B columns (head c < G, the rest zero), A row c of key sub-tile s is key
//   8 (c / 4) + 4 s + c % 4, so output lane (gq, c) = (lane / 16, lane % 16)
//   holds keys 8 gq .. 8 gq + 7 of head c: the B operand layout of the P.V
//   step. Products kh.qh + kh.ql + kl.qh (hi/lo splits, fp32 accumulate).
// * Softmax in base 2 (scores scaled by log2(e) / sqrt(hd)), reductions
//   over the four lane groups.
// * O^T += V^T P^T: one k-step over the tile's keys per 16 dims, A = 16
//   bytes of a V^T row per plane.
// The waves' states merge through LDS into the block's (m, l, o) per head,
// stored agent-coherently for the combining block (the last to arrive on
// the kv head's counter); a context of one block is written out directly.
// Key P (this step's) is not in the planes yet: the block holding it
// normalises and rotates the key (QK-norm, RoPE) and reads the value row
// from the fp32/bf16 cache, patches them into the operands of the last
// tile (keys past P zeroed), and writes them to the cache and the planes.
constexpr int kD2Tile = 32;     // keys per wave step
// Buffer descriptor word 3 for raw (untyped, unswizzled) buffer loads on
// gfx9-family GPUs: 32-bit data format, no index/stride.
constexpr int kRsrcWord3 = 0x00020000;
// Tiles per block, at least: fewer, larger chunks beat more partial
// results to combine at short contexts; a context of up to this many tiles
// is one block per kv head, whose result is the output (no combine).
constexpr int kD2MinTiles = 2;

// Tiles a wave holds in registers at once (128 VGPRs per tile with the
// hi and lo planes, 64 with hi only).
template <bool B16>
constexpr int kD2Tpw = B16 ? 4 : 2;

// Blocks per kv head (nb <= max_blocks) and tiles per block (tpb) for
// `total` keys: as many blocks as allowed, each a whole number of tiles.
__host__ __device__ inline void decode_mfma_split(int total, int max_blocks, int& nb, int& tpb) {
  const int nt = (total + kD2Tile - 1) / kD2Tile;
  const int per = (nt + max_blocks - 1) / max_blocks;
  tpb = per > kD2MinTiles ? per : kD2MinTiles;
  nb = (nt + tpb - 1) / tpb;
}

__device__ __forceinline__ void split8v(const float (&x)[8], bf16x8& hi, bf16x8& lo) {
  uint32_t h[4], l[4];
#pragma unroll
  for (int e = 0; e < 4; e++) split2(x[2 * e], x[2 * e + 1], h[e], l[e]);
  hi = __builtin_bit_cast(bf16x8, (uint4){h[0], h[1], h[2], h[3]});
  lo = __builtin_bit_cast(bf16x8, (uint4){l[0], l[1], l[2], l[3]});
}

// NW wavefronts per block: 4 (one per SIMD, kD2Tpw tiles each in flight)
// or 8 (two per SIMD, half as many tiles each: the same tiles in flight per
// block, and each SIMD interleaves two waves' chains of score MFMAs,
// softmax and value MFMAs).
template <int HD, int GW, bool B16, int NW>
__global__ __launch_bounds__(NW * WAVE) void attn_decode_mfma_kernel(AttnParams p) {
  constexpr int NT = NW * WAVE;
  constexpr int NKK = (HD + 31) / 32;  // 32-dim k-steps of S
  constexpr int DJ = HD / 16;          // 16-dim row blocks of O^T
  constexpr int PER = (HD + WAVE - 1) / WAVE;
  constexpr int MAXV = (kDecMaxG + 1 + NW - 1) / NW;  // head vectors per wave in the prologue
  static_assert((NW == 4 || NW == 8) && kD2Tile == 32, "four or eight waves, 32-key tiles");
  __shared__ __attribute__((aligned(16))) float qs[kDecMaxG * HD];  // normalised, rotated queries
  __shared__ __attribute__((aligned(16))) float kn[HD];             // this step's key
  __shared__ float vn[HD];                                          // this step's value
  __shared__ float mo[NW][kDecMaxG][HD];                            // per-wave outputs
  __shared__ float ml[NW][kDecMaxG][2];                             // per-wave (m, l)
  __shared__ int flag;

  const int blk = blockIdx.x, g = blockIdx.y;
  const int G = p.q_heads / p.kv_heads;
  const int P = *p.pos, total = P + 1;
  int nb, tpb;
  decode_mfma_split(total, p.splits, nb, tpb);
  if (blk >= nb) return;  // not counted: the last block waits for nb arrivals
  const int nt = (total + kD2Tile - 1) / kD2Tile;
  const int t0 = blk * tpb, t1 = min(nt, t0 + tpb);
  const bool has_new = t1 == nt;  // the block holding key P (in tile nt - 1)
  const int tid = threadIdx.x, lane = tid % WAVE, gq = lane / 16, c = lane % 16;
  const int wave = __builtin_amdgcn_readfirstlane(tid / WAVE);  // uniform: tile choices are scalar
  const size_t krow0 = (size_t)g * p.ctx * HD;
  const size_t vrow0 = (size_t)g * HD * p.ctx_pad;

  // Prologue loads, in the order they are needed: the raw q (and new k)
  // vectors, norm weights and the rotation of position P; the new value;
  // then the first two tiles of operands. Out-of-range vector loads read a
  // valid element and are discarded.
  const float* cs = p.rope + (size_t)P * HD;
  const int hp = lane * p.pair_stride;
  const int hq = hp < p.pair_bound ? hp : 0;
  float xv[MAXV][PER], wv[MAXV][PER], fr[MAXV], fi[MAXV];
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
  float vraw = 0.0f;
  if (has_new && tid < HD) vraw = cache_at<B16>(p.vcache, ((size_t)g * p.ctx + P) * HD + tid);

  // Tile operands, straight from HBM into registers in the MFMA operand
  // layouts (buffer loads: 32-bit offsets from the kv head's plane base).
  // A wave holds up to TPW tiles at once; its first TPW tiles are requested
  // here, before the queries are processed, the rest a round at a time.
  struct Regs {
    bf16x8 kh[2][NKK], kl[2][NKK], vh[DJ], vl[DJ];
  };
  const unsigned kbytes = (unsigned)((size_t)p.ctx * HD * 2), vbytes = (unsigned)((size_t)HD * p.ctx_pad * 2);
  const __amdgpu_buffer_rsrc_t rkh = __builtin_amdgcn_make_buffer_rsrc((void*)(p.khi + krow0), 0, kbytes, kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rkl = __builtin_amdgcn_make_buffer_rsrc((void*)(p.klo + krow0), 0, kbytes, kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rvh = __builtin_amdgcn_make_buffer_rsrc((void*)(p.vthi + vrow0), 0, vbytes, kRsrcWord3);
  const __amdgpu_buffer_rsrc_t rvl = __builtin_amdgcn_make_buffer_rsrc((void*)(p.vtlo + vrow0), 0, vbytes, kRsrcWord3);
  auto ld = [](__amdgpu_buffer_rsrc_t r, unsigned off) {
    return __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0));
  };
  auto load = [&](int it, Regs& r) {
    const int key0 = it * kD2Tile;
#pragma unroll
    for (int s = 0; s < 2; s++) {
      const int key = min(key0 + 8 * (c >> 2) + 4 * s + (c & 3), P);  // rows past P: masked
#pragma unroll
      for (int kk = 0; kk < NKK; kk++) {
        const int d = 32 * kk + 8 * gq;
        if (HD >= 32 || d < HD) {  // head_dim 16: dims 16..31 of the k-step are zero
          const unsigned off = (unsigned)(key * HD + d) * 2u;
          r.kh[s][kk] = ld(rkh, off);
          if (!B16) r.kl[s][kk] = ld(rkl, off);
        } else {
          r.kh[s][kk] = bf16x8{};
          r.kl[s][kk] = bf16x8{};
        }
      }
    }
#pragma unroll
    for (int dj = 0; dj < DJ; dj++) {  // key0 + 32 <= ctx_pad
      const unsigned off = (unsigned)((16 * dj + c) * p.ctx_pad + key0 + 8 * gq) * 2u;
      r.vh[dj] = ld(rvh, off);
      if (!B16) r.vl[dj] = ld(rvl, off);
    }
  };
  constexpr int TPW = NW == 4 ? kD2Tpw<B16> : kD2Tpw<B16> / 2;
  const int first = t0 + wave;                                 // tiles first, first + 4, ...
  const int cnt = first < t1 ? (t1 - first + NW - 1) / NW : 0;  // of this wave
  Regs r[TPW];
#pragma unroll
  for (int j = 0; j < TPW; j++)
    if (j < cnt) load(first + j * NW, r[j]);

#pragma unroll
  for (int j = 0; j < MAXV; j++) {
    const int v = wave + j * NW;
    if (v == G)  // this step's key, rounded as a bf16 cache holds it
      norm_rope_regs<HD, B16>(xv[j], wv[j], p.kn != nullptr, p.eps, fr[j], fi[j], p.pair_bound,
                              p.pair_offset, p.pair_stride, kn);
    else if (v < G)
      norm_rope_regs<HD>(xv[j], wv[j], p.qn != nullptr, p.eps, fr[j], fi[j], p.pair_bound, p.pair_offset,
                         p.pair_stride, qs + v * HD);
  }
  if (has_new && tid < HD) vn[tid] = vraw;
  __syncthreads();

  // B operands (dims 32 kk + 8 gq .. + 7 of a head): column c < 8 holds
  // head c's hi part, column c + 8 its lo part (qb); qb2 the hi parts only
  // (for the K lo plane). Columns of heads >= G are zero.
  const int hc = c & 7;
  const bool lo_col = c >= 8;
  bf16x8 qb[NKK], qb2[NKK];
#pragma unroll
  for (int kk = 0; kk < NKK; kk++) {
    const int d = 32 * kk + 8 * gq;
    float x[8];
    if (hc < G && (HD >= 32 || d < HD)) {
      const f32x4 a = *(const f32x4*)(qs + hc * HD + d), b = *(const f32x4*)(qs + hc * HD + d + 4);
      x[0] = a[0]; x[1] = a[1]; x[2] = a[2]; x[3] = a[3]; x[4] = b[0]; x[5] = b[1]; x[6] = b[2]; x[7] = b[3];
    } else {
#pragma unroll
      for (int e = 0; e < 8; e++) x[e] = 0.0f;
    }
    bf16x8 h, lo;
    split8v(x, h, lo);
    qb[kk] = lo_col ? lo : h;
    qb2[kk] = lo_col ? bf16x8{} : h;
  }

  const float sl2 = 1.44269504088896341f / sqrtf((float)HD);
  float m = -INFINITY, l = 0.0f;
  f32x4 o[DJ];
#pragma unroll
  for (int dj = 0; dj < DJ; dj++) o[dj] = f32x4{0.f, 0.f, 0.f, 0.f};

  // The last tile's operands get key P (K row, V^T column) and zeros for
  // the V^T entries of keys past P.
  auto patch = [&](Regs& r, int key0) {
#pragma unroll
    for (int s = 0; s < 2; s++) {
      if (key0 + 8 * (c >> 2) + 4 * s + (c & 3) == P) {
#pragma unroll
        for (int kk = 0; kk < NKK; kk++) {
          const int d = 32 * kk + 8 * gq;
          if (HD >= 32 || d < HD) {
            float x[8];
#pragma unroll
            for (int e = 0; e < 8; e++) x[e] = kn[d + e];
            split8v(x, r.kh[s][kk], r.kl[s][kk]);
          }
        }
      }
    }
    const int at = P - key0 - 8 * gq;  // the lane's V^T element holding key P
    if (at < 8) {  // key P or keys past it among the lane's eight
      typedef unsigned short u16x8 __attribute__((ext_vector_type(8)));
#pragma unroll
      for (int dj = 0; dj < DJ; dj++) {
        u16x8 h = __builtin_bit_cast(u16x8, r.vh[dj]), lo = __builtin_bit_cast(u16x8, r.vl[dj]);
        uint32_t nh, nl;
        split2(vn[16 * dj + c], 0.0f, nh, nl);
#pragma unroll
        for (int e = 0; e < 8; e++) {
          h[e] = e < at ? h[e] : e == at ? (unsigned short)nh : (unsigned short)0;
          lo[e] = e < at ? lo[e] : e == at ? (unsigned short)nl : (unsigned short)0;
        }
        r.vh[dj] = __builtin_bit_cast(bf16x8, h);
        r.vl[dj] = __builtin_bit_cast(bf16x8, lo);
      }
    }
  };

  auto step = [&](Regs& r, int it) {
    const int key0 = it * kD2Tile;
    if (it == nt - 1) patch(r, key0);
    // column c: kh.qh + kl.qh (c < 8) or kh.ql (c >= 8); columns c and
    // c ^ 8 summed (a rotation by 8 within each row of 16 lanes) give the
    // score of head c & 7 in both
    f32x4 sc[2];
#pragma unroll
    for (int s = 0; s < 2; s++) {
      sc[s] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < NKK; kk++) {
        sc[s] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(r.kh[s][kk], qb[kk], sc[s], 0, 0, 0);
        if (!B16) sc[s] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(r.kl[s][kk], qb2[kk], sc[s], 0, 0, 0);
      }
    }
    float pv[8];
    float mx = -INFINITY;
    const bool full = key0 + kD2Tile - 1 <= P;
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const float x = sc[j >> 2][j & 3];
      const float sum = (x + dpp_ror8(x)) * sl2;  // every lane (the DPP reads lane c ^ 8)
      const float v = full || key0 + 8 * gq + j <= P ? sum : -INFINITY;
      pv[j] = v;
      mx = fmaxf(mx, v);
    }
    mx = fmaxf(mx, xor16_max(mx));
    mx = fmaxf(mx, xor32_max(mx));
    const float mn = fmaxf(m, mx);  // finite: key key0 <= P is in every tile
    const float corr = __builtin_amdgcn_exp2f(m - mn);
    float rs = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; j++) {
      const float e = __builtin_amdgcn_exp2f(pv[j] - mn);
      pv[j] = e;
      rs += e;
    }
    rs = xor16_sum(rs);
    rs = xor32_sum(rs);
    l = l * corr + rs;
    m = mn;
    // P^T columns as the queries': hi in c < 8, lo in c >= 8 (pb), hi only
    // for the V lo plane (pb2); column c ^ 8 is folded in after the loop
    bf16x8 ph, pl;
    split8v(pv, ph, pl);
    const bf16x8 pb = lo_col ? pl : ph, pb2 = lo_col ? bf16x8{} : ph;
#pragma unroll
    for (int dj = 0; dj < DJ; dj++) {
      o[dj] *= corr;
      o[dj] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(r.vh[dj], pb, o[dj], 0, 0, 0);
      if (!B16) o[dj] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(r.vl[dj], pb2, o[dj], 0, 0, 0);
    }
  };

  for (int b = 0; b < cnt; b += TPW) {
    if (b > 0) {
#pragma unroll
      for (int j = 0; j < TPW; j++)
        if (b + j < cnt) load(first + (b + j) * NW, r[j]);
    }
#pragma unroll
    for (int j = 0; j < TPW; j++)
      if (b + j < cnt) step(r[j], first + (b + j) * NW);
  }

  // Merge the waves (a wave without tiles has m = -inf, l = 0, o = 0);
  // head c's output is the sum of columns c and c + 8.
#pragma unroll
  for (int dj = 0; dj < DJ; dj++)
#pragma unroll
    for (int e = 0; e < 4; e++) o[dj][e] += dpp_ror8(o[dj][e]);
  if (c < G) {
#pragma unroll
    for (int dj = 0; dj < DJ; dj++)
#pragma unroll
      for (int e = 0; e < 4; e++) mo[wave][c][16 * dj + 4 * gq + e] = o[dj][e];
    if (gq == 0) {
      ml[wave][c][0] = m;
      ml[wave][c][1] = l;
    }
  }
  __syncthreads();
  for (int i = tid; i < G * HD; i += NT) {
    const int h = i / HD, d = i % HD;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; w++) M = fmaxf(M, ml[w][h][0]);
    float O = 0.0f, Lb = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; w++) {
      const float f = __builtin_amdgcn_exp2f(ml[w][h][0] - M);
      O = fmaf(f, mo[w][h][d], O);
      Lb = fmaf(f, ml[w][h][1], Lb);
    }
    if (nb == 1) {  // the whole context: the block's result is the output
      p.out[(size_t)(g * G + h) * HD + d] = O / Lb;
      continue;
    }
    float* part = p.partial + ((size_t)(g * G + h) * p.splits + blk) * (HD + 2);
    cstore(part + 2 + d, O);
    if (d == 0) {
      cstore(part, M);
      cstore(part + 1, Lb);
    }
  }
  if (has_new && tid < HD) {  // row P of the cache and its planes, read by later steps
    const size_t at = ((size_t)g * p.ctx + P) * HD + tid;
    const float k = kn[tid], v = vn[tid];
    if (B16) ((uint16_t*)p.kcache_w)[at] = f32_to_bf16_any(k);  // exact: kn is rounded
    else p.kcache_w[at] = k;
    uint32_t hk, lk, hv, lv;
    split2(k, 0.0f, hk, lk);
    split2(v, 0.0f, hv, lv);
    // the planes are this kernel's operands (read-only above); row P is
    // read by no block of this launch
    ((uint16_t*)p.khi)[at] = (uint16_t)hk;
    ((uint16_t*)p.klo)[at] = (uint16_t)lk;
    const size_t vt = vrow0 + (size_t)tid * p.ctx_pad + P;
    ((uint16_t*)p.vthi)[vt] = (uint16_t)hv;
    ((uint16_t*)p.vtlo)[vt] = (uint16_t)lv;
  }
  if (nb == 1) return;
  // Hand-off to the combining block. Partials are written and read only by
  // agent-scope relaxed atomic accesses (sc1: written through to, and read
  // from, the agent's coherence point, never from a non-coherent L2 line),
  // and this wait makes every one of the block's stores complete before the
  // counter increment is issued; the combining block issues its loads after
  // its own increment has returned. That is the AMDGPU release/acquire
  // sequence without its cache write-back and invalidate, which only
  // non-atomic accesses need. (An acq_rel increment adds both: +1.3 us per
  // launch at 640 positions, +2.6 us at 2176.)
  compiler_fence();
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (tid == 0) {
    const unsigned done = __hip_atomic_fetch_add(p.counters + g, 1u, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
    flag = done == (unsigned)(nb - 1);
  }
  __syncthreads();
  if (!flag) return;
  compiler_fence();

  // Last block of kv head g: wave w combines heads w*GW .., lane c holding
  // block c's weight (scores in base 2). Every block partial of the lane's
  // output dims (of all the wave's heads when they fit in registers) is
  // loaded before the first is used, 8 blocks per batch up to nb, then
  // summed in block order:
  //   att = sum_c 2^(m_c - M) o_c / sum_c 2^(m_c - M) l_c,  M = max_c m_c,
  // and the counter is reset for the next launch.
  constexpr int DPL = HD >= WAVE ? HD / WAVE : 1;
  constexpr int CB = 8;
  constexpr int HB = GW * DPL <= 2 ? GW : 1;
  const int dd = min(lane * DPL, HD - DPL);
  const bool ok = lane < nb;
#pragma unroll
  for (int j0 = 0; j0 < GW; j0 += HB) {
    if (wave * GW + j0 >= G) break;
    float mc[HB], lc[HB], x[HB][kDecMaxChunks][DPL];
#pragma unroll
    for (int j = 0; j < HB; j++) {
      const float* base = p.partial + (size_t)(g * G + min(wave * GW + j0 + j, G - 1)) * p.splits * (HD + 2);
      mc[j] = ok ? cload(base + (size_t)lane * (HD + 2)) : -INFINITY;
      lc[j] = ok ? cload(base + (size_t)lane * (HD + 2) + 1) : 0.0f;
    }
#pragma unroll
    for (int j = 0; j < HB; j++) {
      const float* base = p.partial + (size_t)(g * G + min(wave * GW + j0 + j, G - 1)) * p.splits * (HD + 2);
#pragma unroll
      for (int b = 0; b < kDecMaxChunks / CB; b++) {
        if (b * CB < nb) {
#pragma unroll
          for (int i = 0; i < CB; i++) {
            const float* src = base + (size_t)min(b * CB + i, nb - 1) * (HD + 2) + 2 + dd;
            if constexpr (DPL == 2) {
              const float2 f = cload2(src);
              x[j][b * CB + i][0] = f.x;
              x[j][b * CB + i][1] = f.y;
            } else {
#pragma unroll
              for (int d = 0; d < DPL; d++) x[j][b * CB + i][d] = cload(src + d);
            }
          }
        }
      }
    }
#pragma unroll
    for (int j = 0; j < HB; j++) {
      const int h = wave * GW + j0 + j;
      if (h >= G) break;
      const float M = wave_peak(mc[j]);
      const float w = ok ? __builtin_amdgcn_exp2f(mc[j] - M) : 0.0f;
      const float W = wave_total(w * lc[j]);
      float oo[DPL];
#pragma unroll
      for (int d = 0; d < DPL; d++) oo[d] = 0.0f;
#pragma unroll
      for (int b = 0; b < kDecMaxChunks / CB; b++) {
        if (b * CB < nb) {
#pragma unroll
          for (int i = 0; i < CB; i++) {
            const float wc = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w), b * CB + i));
#pragma unroll
            for (int d = 0; d < DPL; d++) oo[d] = fmaf(wc, x[j][b * CB + i][d], oo[d]);
          }
        }
      }
      if (lane * DPL < HD) {
#pragma unroll
        for (int d = 0; d < DPL; d++) p.out[(size_t)(g * G + h) * HD + lane * DPL + d] = oo[d] / W;
      }
    }
  }
  if (tid == 0) __hip_atomic_store(p.counters + g, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

}  // namespace

// Wavefronts per decode attention block: 8 by default, 4 with
// STRASGPT_DECODE_ATTN_WAVES=4. Eight (two per SIMD, one fp32 tile each)
// against four (one per SIMD, two tiles each), stand-alone at the
// Mistral-Small-24B / Llama-3.1-8B head shape (32 query heads, 8 kv heads,
// head_dim 128): 9.04 -> 8.78 us at 600 positions, 11.50 -> 11.28 at 2112,
// 19.87 -> 18.77 at 8300 (24-32 blocks per kv head within 0.2 us).
int attention_decode_waves() {
  if (const char* v = getenv("STRASGPT_DECODE_ATTN_WAVES")) {
    const int n = atoi(v);
    if (n != 4 && n != 8) ST_DIE("STRASGPT_DECODE_ATTN_WAVES must be 4 or 8");
    return n;
  }
  return 8;
}

// Blocks per kv head, at most: up to 256 blocks, one per CU (a block holds
// each SIMD's register file), and at most one combine lane each.
int attention_decode_chunks(int kv_heads) {
  // STRASGPT_DECODE_ATTN_CHUNKS: blocks per kv head at most (1-64), for
  // sweeps; by default one block per CU over the kv heads
  if (const char* v = getenv("STRASGPT_DECODE_ATTN_CHUNKS")) {
    const int n = atoi(v);
    if (n < 1 || n > kDecMaxChunks) ST_DIE("STRASGPT_DECODE_ATTN_CHUNKS must be 1-64");
    return n;
  }
  return std::max(1, std::min(kDecMaxChunks, 256 / std::max(1, kv_heads)));
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
#define X3_ATTR(HD)                                                                  \
  HIP_CHECK(hipFuncSetAttribute((const void*)attn_prefill_x3_kernel<HD, 1>,          \
                                hipFuncAttributeMaxDynamicSharedMemorySize,          \
                                X3Lds<HD>::bytes));                                  \
  HIP_CHECK(hipFuncSetAttribute((const void*)attn_prefill_x3_kernel<HD, 2>,          \
                                hipFuncAttributeMaxDynamicSharedMemorySize,          \
                                X3Lds<HD>::bytes));
  X3_ATTR(16)
  X3_ATTR(32)
  X3_ATTR(64)
  X3_ATTR(128)
#undef X3_ATTR
}

// STRASGPT_PREFILL_ATTN=fp32 selects the fp32 matrix-core kernel; the
// default is the split bf16 one (about 3x faster at long contexts), with 32
// queries per wavefront where the grid of 128-query blocks still fills two
// blocks per CU, else 16 (x3-16 / x3-32 force one of them).
int prefill_attn_mode() {
  const char* e = getenv("STRASGPT_PREFILL_ATTN");
  if (!e || !*e || !strcmp(e, "x3")) return 0;
  if (!strcmp(e, "fp32")) return 1;
  if (!strcmp(e, "x3-16")) return 2;
  if (!strcmp(e, "x3-32")) return 3;
  ST_DIE("STRASGPT_PREFILL_ATTN must be x3, x3-16, x3-32 or fp32");
}

void attention_prefill(const AttnParams& p, hipStream_t s) {
  attention_prefill_variant(p, prefill_attn_mode(), s);
}

void attention_split_rows(const float* kcache, const float* vcache, uint16_t* khi, uint16_t* klo,
                          uint16_t* vthi, uint16_t* vtlo, int kv_heads, int ctx, int ctx_pad, int hd,
                          int r0, int r1, int kv_bf16, hipStream_t s) {
  if (r0 % 32 || r0 < 0 || r1 > ctx || ctx_pad % 32 || ctx_pad < ctx)
    ST_DIE("attention_split_rows: rows must start at a multiple of 32 and stay in the cache");
  if (r1 <= r0) return;
  const dim3 grid((r1 - r0 + 31) / 32, kv_heads);
  switch (hd) {
#define SPLIT_CASE(HD)                                                                                \
  case HD:                                                                                            \
    if (kv_bf16)                                                                                      \
      hipLaunchKernelGGL((split_rows_kernel<HD, true>), grid, dim3(256), 0, s, kcache, vcache, khi, klo, \
                         vthi, vtlo, ctx, ctx_pad, r0, r1);                                           \
    else                                                                                              \
      hipLaunchKernelGGL((split_rows_kernel<HD, false>), grid, dim3(256), 0, s, kcache, vcache, khi, klo, \
                         vthi, vtlo, ctx, ctx_pad, r0, r1);                                           \
    break;
    SPLIT_CASE(16)
    SPLIT_CASE(32)
    SPLIT_CASE(64)
    SPLIT_CASE(128)
#undef SPLIT_CASE
    default: ST_DIE("attention supports head_dim 16, 32, 64 or 128");
  }
  HIP_CHECK(hipGetLastError());
}

void attention_prefill_variant(const AttnParams& p, int variant, hipStream_t s) {
  if (p.T <= 0 || p.q_heads % p.kv_heads) ST_DIE("bad attention shape");
  if (!p.out_hi && !p.out) ST_DIE("prefill attention writes bf16 planes (out_hi) or fp32 rows (out)");
  if (variant == 0 && (!p.khi || !p.klo || !p.vthi || !p.vtlo || p.ctx_pad % 32 || p.ctx_pad < p.ctx))
    ST_DIE("split-bf16 prefill attention needs the cache's bf16 planes");
  if (variant < 0 || variant > 3) ST_DIE("prefill attention variant is 0 (split bf16), 1 (fp32), 2 or 3");
  if (variant == 1 && p.kv_bf16) ST_DIE("the fp32 prefill attention kernel reads an fp32 KV cache only");
  const bool fp32 = variant == 1;
  // split bf16: 32 queries per wave when 128-query blocks give 2 per CU
  const bool wide = variant == 3 || (variant == 0 && (long)((p.T + 2 * PQ - 1) / (2 * PQ)) * p.q_heads >= 512);
  const int nqb = (p.T + (wide ? 2 * PQ : PQ) - 1) / (wide ? 2 * PQ : PQ);
  // x3: (heads, query blocks), longest ranges of every head first; fp32: (query blocks, heads)
  const dim3 grid = fp32 ? dim3(nqb, p.q_heads) : dim3(p.q_heads, nqb);
  switch (p.hd) {
#define PREFILL_CASE(HD)                                                                         \
  case HD:                                                                                       \
    if (fp32)                                                                                    \
      hipLaunchKernelGGL(attn_prefill_mfma_kernel<HD>, grid, dim3(256), 4 * PK * HD * sizeof(float), s, p); \
    else if (wide)                                                                               \
      hipLaunchKernelGGL((attn_prefill_x3_kernel<HD, 2>), grid, dim3(256), X3Lds<HD>::bytes, s, p); \
    else                                                                                         \
      hipLaunchKernelGGL((attn_prefill_x3_kernel<HD, 1>), grid, dim3(256), X3Lds<HD>::bytes, s, p); \
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
  if (!p.khi || !p.klo || !p.vthi || !p.vtlo || p.ctx_pad % 32 || p.ctx_pad < p.ctx)
    ST_DIE("decode attention needs the cache's bf16 planes");
  if (p.pair_stride < 1 || (p.pair_bound + p.pair_stride - 1) / p.pair_stride > WAVE ||
      p.pair_bound - p.pair_stride + p.pair_offset >= p.hd)
    ST_DIE("decode attention: RoPE pairs must fit one per lane within the head");
  const dim3 grid(p.splits, p.kv_heads);
  const int nw = attention_decode_waves();
  const bool two = nw == 4 && G > 4;  // the combine: two query heads per wave
  switch (p.hd) {
#define DECODE2_LAUNCH(HD, GW, NW)                                                                        \
  if (p.kv_bf16)                                                                                          \
    hipLaunchKernelGGL((attn_decode_mfma_kernel<HD, GW, true, NW>), grid, dim3(NW * WAVE), 0, s, p);     \
  else                                                                                                    \
    hipLaunchKernelGGL((attn_decode_mfma_kernel<HD, GW, false, NW>), grid, dim3(NW * WAVE), 0, s, p);
#define DECODE2_CASE(HD)        \
  case HD:                      \
    if (nw == 8) {              \
      DECODE2_LAUNCH(HD, 1, 8)  \
    } else if (two) {           \
      DECODE2_LAUNCH(HD, 2, 4)  \
    } else {                    \
      DECODE2_LAUNCH(HD, 1, 4)  \
    }                           \
    break;
    DECODE2_CASE(16)
    DECODE2_CASE(32)
    DECODE2_CASE(64)
    DECODE2_CASE(128)
#undef DECODE2_CASE
#undef DECODE2_LAUNCH
    default: ST_DIE("attention supports head_dim 16, 32, 64 or 128");
  }
  HIP_CHECK(hipGetLastError());
}

}  // namespace sg
