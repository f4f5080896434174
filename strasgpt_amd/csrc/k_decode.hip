// Persistent decode step on gfx950: one launch per generated token of a
// dense model (reference transformer_predict with one token,
// source/transformer.c:1186-1602, then the greedy argmax of
// source/sampler.c).
//
// The grid is one 512-thread block per compute unit, all resident at once
// (cooperative launch; the LDS request keeps two blocks off one CU). Block
// 0 only coordinates the grid barriers (grid_sync.h) and reduces the
// argmax; the other blocks are workers. The step is a sequence of phases
// separated by grid barriers:
//
//   per layer: QKV GEMV (RMSNorm prologue; layer 0 embeds the token)
//              attention over (kv head, key chunk) items, QK-norm + RoPE,
//                writes the new key/value row into the cache
//              combine of the chunk partials per head
//              O GEMV + residual
//              gate/up GEMV + SwiGLU (RMSNorm prologue)
//              down GEMV + residual
//   then:      logits GEMV (final RMSNorm prologue) + per-block argmax
//              argmax of the block winners, *next, seq, *pos += 1
//
// Each GEMV phase gives every worker `rb` consecutive output rows, cut
// into S slices per row; the block's 8 waves take slices round-robin and
// walk them with 128-bit non-temporal weight loads (8 bf16 per lane, 16
// loads per lane in flight, double-buffered in registers). A worker arrives
// at a barrier as soon as its stores are complete, then issues the next
// phase's first batch of weight loads (attention: its first K/V tile, rows
// from earlier steps) and only then waits, so HBM keeps streaming while the
// barrier completes. Slice sums are reduced per row in LDS in slice order
// (deterministic), then the epilogue runs one thread per row.
//
// Activations crossing blocks (x, q/k/v, attention partials and outputs,
// SwiGLU output, argmax winners) are written and read with agent-coherent
// accesses only; the barriers carry no cache fences.
//
// Algorithmic bytes per launch: every bf16 weight once (L x (qkv + o +
// gate + up + down) + logits matrix), plus 2 x kv_heads x (pos+1) x hd x 4
// bytes of KV cache per layer.
#include <math.h>

#include "device_common.h"
#include "grid_sync.h"
#include "hip_check.h"
#include "kernels.h"

namespace sg {

namespace {

constexpr int kT = kDecodeThreads;  // 512
constexpr int kW = kT / WAVE;       // 8 waves
constexpr int kU = 8;  // weight loads per lane per batch (4 per matrix for a pair)
constexpr int kMaxG = 8;            // q heads per kv head
constexpr int kMinChunk = 16;       // keys per attention item, at least
constexpr size_t kMinLds = 81 * 1024;  // more than half of a CU's LDS

// Parameters are read from a copy in LDS (made at kernel start) and made
// wave-uniform at each use: no parameter stays live in scalar registers
// across the step (the step's code is large; long-lived scalars spill), and
// the reads never queue behind the weight stream.
__device__ __forceinline__ int U(int v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ unsigned U(unsigned v) {
  return (unsigned)__builtin_amdgcn_readfirstlane((int)v);
}
__device__ __forceinline__ float U(float v) {
  return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(v)));
}
__device__ __forceinline__ size_t U(size_t v) {
  const unsigned lo = U((unsigned)v), hi = U((unsigned)(v >> 32));
  return ((size_t)hi << 32) | lo;
}
template <typename T>
__device__ __forceinline__ T* U(T* v) {
  return (T*)U((size_t)v);
}
__device__ __forceinline__ DecodeGemvPlan U(const DecodeGemvPlan& v) {
  return DecodeGemvPlan{U(v.rb), U(v.S), U(v.ks)};
}
constexpr int kParamFloats = 128;  // LDS floats reserved for the parameter copy
static_assert(sizeof(DecodeParams) <= kParamFloats * sizeof(float), "parameter block");

// ---------------------------------------------------------------- GEMV --
//
// One code path serves every GEMV phase (the kernel is large, and one copy
// of its streaming loop stays in the instruction cache): the matrix pair of
// gate/up (`dual`), the epilogue and the input staging are run-time
// choices.

enum Epilogue { EPI_QKV, EPI_RESIDUAL, EPI_SWIGLU, EPI_LOGITS };

struct Job {
  const uint16_t* w;
  const uint16_t* w2;  // second matrix of a pair, or null
  int K, row0, rows, log2s, ks, it, items;
  unsigned safe;  // element offset loaded by masked lanes (a valid address)
};

__device__ __forceinline__ Job make_job(const uint16_t* w, const uint16_t* w2, int N, int K,
                                        const DecodeGemvPlan& pl, int worker) {
  Job j;
  j.w = w;
  j.w2 = w2;
  j.K = K;
  j.row0 = worker * pl.rb;
  j.rows = max(0, min(pl.rb, N - j.row0));
  j.log2s = 31 - __builtin_clz(pl.S);
  j.ks = pl.ks;
  j.it = (pl.ks + WAVE - 1) / WAVE;
  j.safe = (unsigned)min(j.row0, N - 1) * K + min((int)(threadIdx.x % WAVE) * 8, K - 8);
  const int wave = threadIdx.x / WAVE, slices = j.rows << j.log2s;
  j.items = slices > wave ? (slices - wave + kW - 1) / kW * j.it : 0;
  return j;
}

// Position in a wave's item sequence: item n is iteration i (of it) of the
// wave's slice sl (block slice wave + 8 sl).
struct Cursor {
  int n, sl, i;
};

struct Batch {
  uint4 a[kU];
};

// Element offset of the cursor's item for this lane, or j.safe when the
// lane is past its slice; advances the cursor. Call only while c.n < items.
// (Matrices have fewer than 2^32 elements: offsets are 32-bit.)
__device__ __forceinline__ unsigned item_offset(const Job& j, Cursor& c, int lane, int wave) {
  const int q = wave + kW * c.sl;
  const int row = j.row0 + (q >> j.log2s), part = q & ((1 << j.log2s) - 1);
  const int ch = c.i * WAVE + lane, col = (part * j.ks + ch) * 8;
  const unsigned off = (ch < j.ks && col < j.K) ? (unsigned)row * j.K + col : j.safe;
  c.n++;
  if (++c.i == j.it) {
    c.i = 0;
    c.sl++;
  }
  return off;
}

// Issues exactly kU loads: up to kU items of one matrix, or up to kU/2
// items of each matrix of a pair (slots kU/2 + u hold the second matrix's
// item u). Slots past the wave's work load `safe` (lines already in flight).
__device__ __forceinline__ void load_batch(const Job& j, Cursor& c, Batch& B) {
  const int lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  const bool dual = j.w2 != nullptr;
  const int per = dual ? kU / 2 : kU;
#pragma unroll
  for (int u = 0; u < kU / 2; u++) {
    const unsigned off = c.n < j.items ? item_offset(j, c, lane, wave) : j.safe;
    B.a[u] = load_nt_u4(j.w + off);
    if (dual) B.a[u + kU / 2] = load_nt_u4(j.w2 + off);
  }
  if (per == kU) {
#pragma unroll
    for (int u = kU / 2; u < kU; u++) {
      const unsigned off = c.n < j.items ? item_offset(j, c, lane, wave) : j.safe;
      B.a[u] = load_nt_u4(j.w + off);
    }
  }
}

__device__ __forceinline__ void mul_batch(const Job& j, Cursor& c, const Batch& B, const float* xs,
                                          float& acc, float& acc2, float* part1, float* part2) {
  const int lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  const bool dual = j.w2 != nullptr;
  const int per = dual ? kU / 2 : kU;
#pragma unroll
  for (int u = 0; u < kU; u++) {
    if (u < per && c.n < j.items) {
      const int q = wave + kW * c.sl;
      const int part = q & ((1 << j.log2s) - 1);
      const int ch = c.i * WAVE + lane, col = (part * j.ks + ch) * 8;
      if (ch < j.ks && col < j.K) {
        const float4 x0 = *(const float4*)(xs + col);
        const float4 x1 = *(const float4*)(xs + col + 4);
        acc = dot8(B.a[u], x0, x1, acc);
        if (dual) acc2 = dot8(B.a[(u + kU / 2) % kU], x0, x1, acc2);
      }
      c.n++;
      if (++c.i == j.it) {  // slice done
        const float s1 = wave_sum(acc);
        if (lane == 0) part1[q] = s1;
        if (dual) {
          const float s2 = wave_sum(acc2);
          if (lane == 0) part2[q] = s2;
        }
        acc = 0.0f;
        acc2 = 0.0f;
        c.i = 0;
        c.sl++;
      }
    }
  }
}

// Rest of a GEMV phase after the prefetched first batch `cur` (loader
// cursor `ld` past it), with the input row staged in LDS `xs`: leaves the
// row results (y, and y2 for a pair) for the block's rows r = 0 .. rows-1
// in part1[r] (part2[r]), slice sums added in slice order.
template <typename Mark>
__device__ __forceinline__ void gemv_run(const Job& j, Batch& cur, Cursor ld, const float* xs,
                                         float* part1, float* part2, Mark mark) {
  const bool dual = j.w2 != nullptr;
  const int per = dual ? kU / 2 : kU;
  Cursor cc{0, 0, 0};
  float acc = 0.0f, acc2 = 0.0f;
  const int nb = (j.items + per - 1) / per;
  for (int b = 0; b < nb; b++) {
    Batch nxt;
    const bool more = b + 1 < nb;
    if (more) load_batch(j, ld, nxt);
    mul_batch(j, cc, cur, xs, acc, acc2, part1, part2);
    if (more) cur = nxt;
  }
  __syncthreads();
  mark(3);
  const int S = 1 << j.log2s;
  if (S > 1) {  // slice sums to row results, in slice order
    float y[4], y2[4];
    int n = 0;
    for (int r = threadIdx.x; r < j.rows && n < 4; r += kT, n++) {
      y[n] = 0.0f;
      y2[n] = 0.0f;
      for (int s2 = 0; s2 < S; s2++) {
        y[n] += part1[r * S + s2];
        if (dual) y2[n] += part2[r * S + s2];
      }
    }
    __syncthreads();
    n = 0;
    for (int r = threadIdx.x; r < j.rows && n < 4; r += kT, n++) {
      part1[r] = y[n];
      if (dual) part2[r] = y2[n];
    }
    __syncthreads();
  }
}

// xs[0, n) = src[0, n) read agent-coherent (n even, src 8-byte aligned);
// returns this thread's sum of squares of what it copied. Loads go out in
// batches of 8 x 64 bits per thread before any is used, so the copy costs
// about one memory round trip per 4096 pairs.
__device__ __forceinline__ float stage_coherent(const float* src, int n, float* xs) {
  constexpr int B = 8;
  const unsigned long long* s2 = (const unsigned long long*)src;
  const int pairs = n / 2;
  float ss = 0.0f;
  for (int base = threadIdx.x; base < pairs; base += kT * B) {
    unsigned long long v[B];
#pragma unroll
    for (int i = 0; i < B; i++) {
      const int idx = base + i * kT;
      v[i] = idx < pairs
                 ? __hip_atomic_load(s2 + idx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                 : 0ull;
    }
#pragma unroll
    for (int i = 0; i < B; i++) {
      const int idx = base + i * kT;
      if (idx < pairs) {
        const float a = __uint_as_float((unsigned)v[i]);
        const float b = __uint_as_float((unsigned)(v[i] >> 32));
        *(float2*)(xs + 2 * idx) = make_float2(a, b);
        ss = fmaf(a, a, ss);
        ss = fmaf(b, b, ss);
      }
    }
  }
  return ss;
}

// Input row of a GEMV phase into LDS xs[0, K):
//   emb != null: x = embedding row emb (bf16 -> fp32, exact), this worker
//                also publishing its share of x to `x` (layer 0);
//   otherwise:   x = src read agent-coherent;
// then, when nw != null, xs = RMSNorm(x) with weight nw, else xs = x.
// cap_raw / cap_norm (null, or written by the caller's chosen worker):
// copies of x before and after the RMSNorm.
__device__ __forceinline__ void stage_input(const float* src, const uint16_t* emb, float* x,
                                            int K, const uint16_t* nw, float eps, float* xs,
                                            float* red, int worker, int workers, float* cap_raw,
                                            float* cap_norm) {
  float ss = 0.0f;
  if (emb) {
    const int per = (K + workers - 1) / workers;
    for (int k = threadIdx.x; k < K; k += kT) {
      const float v = bf16_to_f32(gload(emb + k));
      xs[k] = v;
      ss = fmaf(v, v, ss);
      if (k / per == worker) cstore(x + k, v);
    }
  } else {
    ss = stage_coherent(src, K, xs);
  }
  if (cap_raw) {
    __syncthreads();  // xs written by other threads
    for (int k = threadIdx.x; k < K; k += kT) gstore(cap_raw + k, xs[k]);
  }
  if (nw) {
    const float s = rms_scale(block_sum<kT>(ss, red), K, eps);
    for (int k = threadIdx.x; k < K; k += kT) xs[k] = (xs[k] * s) * bf16_to_f32(gload(nw + k));
  }
  if (cap_norm)
    for (int k = threadIdx.x; k < K; k += kT) gstore(cap_norm + k, xs[k]);
  __syncthreads();
}

// ----------------------------------------------------------- attention --

__device__ __forceinline__ void attn_chunks(int total, int max_chunks, int& nch, int& len) {
  nch = min(max_chunks, (total + kMinChunk - 1) / kMinChunk);
  len = (total + nch - 1) / nch;
  nch = (total + len - 1) / len;  // no empty chunk
}

// RMSNorm (optional) + RoPE of one head vector by one wavefront, from the
// agent-coherent q/k/v buffer into LDS `dst`. Same arithmetic as the
// reference (source/transformer.c:1293-1323).
template <int HD>
__device__ __forceinline__ void norm_rope_vec(const float* src, const uint16_t* nw, float eps, const float* cs,
                              int pb, int po, int pst, float* dst) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x % WAVE;
  constexpr int PER = (HD + WAVE - 1) / WAVE;
  float xv[PER];
#pragma unroll
  for (int i = 0; i < PER; i++) xv[i] = lane + i * WAVE < HD ? cload(src + lane + i * WAVE) : 0.0f;
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < PER; i++) {
    if (lane + i * WAVE < HD) {
      dst[lane + i * WAVE] = xv[i];
      ss = fmaf(xv[i], xv[i], ss);
    }
  }
  ss = wave_sum(ss);
  if (nw) {
    const float s = rms_scale(ss, HD, eps);
    for (int e = lane; e < HD; e += WAVE) dst[e] = (dst[e] * s) * bf16_to_f32(gload(nw + e));
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  float r0[4], r1[4];
  int hh[4];
  int cnt = 0;
  for (int i = lane; i * pst < pb; i += WAVE) {
    const int h = i * pst;
    const float fr = gload(cs + h), fi = gload(cs + h + po);
    const float v0 = dst[h], v1 = dst[h + po];
    r0[cnt] = v0 * fr - v1 * fi;
    r1[cnt] = v0 * fi + v1 * fr;
    hh[cnt] = h;
    cnt++;
  }
  __builtin_amdgcn_wave_barrier();
  for (int c = 0; c < cnt; c++) {
    dst[hh[c]] = r0[c];
    dst[hh[c] + po] = r1[c];
  }
}

typedef __attribute__((address_space(3))) void* lds_ptr;

// N consecutive floats from LDS (16-byte aligned when N % 4 == 0, 8-byte
// when N == 2), in the widest reads.
template <int N>
__device__ __forceinline__ void lds_vec(const float* src, float* dst) {
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

// LDS floats used by the attention phase before its K/V tile buffers.
template <int HD>
constexpr int attn_lds_head() { return 10 * HD + kMaxG * 64 + 4 * kMaxG + kT * kMaxG; }

// Rows [t0, t0 + n) (n <= 64) of a kv head's K and V cache, contiguous in
// memory, copied into LDS kt / vt by the global-to-LDS DMA (16 bytes per
// lane; no registers held). The caller waits for vector memory operations
// and syncs the block before reading them.
template <int HD>
__device__ __forceinline__ void dma_kv_tile(const float* kb, const float* vb, int t0, int n,
                                            float* kt, float* vt) {
  const int units = n * HD / 4;
  const int wave = threadIdx.x / WAVE, lane = threadIdx.x % WAVE;
  const float* ks = kb + (size_t)t0 * HD;
  const float* vs = vb + (size_t)t0 * HD;
  for (int u0 = wave * WAVE; u0 < units; u0 += kT) {
    const int u = u0 + lane;
    if (u < units) {
      __builtin_amdgcn_global_load_lds((const void*)(ks + u * 4), (lds_ptr)(kt + u0 * 4), 16, 0, 0);
      __builtin_amdgcn_global_load_lds((const void*)(vs + u * 4), (lds_ptr)(vt + u0 * 4), 16, 0, 0);
    }
  }
}

// Attention work item of a worker: kv head g, key chunk c = [s0, s1).
struct AttnItem {
  bool valid;
  int g, c, s0, s1;
};

__device__ __forceinline__ AttnItem attn_item(const DecodeParams* lp, int P, int worker) {
  int nch, len;
  attn_chunks(P + 1, U(lp->max_chunks), nch, len);
  AttnItem it;
  it.valid = worker < U(lp->kvh) * nch;  // at most one item per worker (host check)
  it.g = worker / nch;
  it.c = worker % nch;
  it.s0 = it.c * len;
  it.s1 = min(P + 1, it.s0 + len);
  return it;
}

// For the G query heads of kv head g: the softmax statistics (max m, sum l)
// and the unnormalised P.V over the item's keys, in tiles of 64 keys with
// an online rescale. The item's first tile was put in flight to LDS
// (dma_kv_tile) before the barrier that precedes this phase; row P, written
// by this step, comes from the new key and value instead.
template <int HD, typename Mark>
__device__ __forceinline__ void attention_phase(const DecodeParams* lp, const DecodeLayer& ly,
                                                int P, const AttnItem& it, float* lds,
                                                Mark mark) {
  constexpr int KP = HD / 8;   // dims per lane for scores (8 lanes per key)
  constexpr int KG = kT / HD;  // key groups for P.V
  if (!it.valid) return;
  const int G = U(lp->qh) / U(lp->kvh);
  float* qs = lds;              // [kMaxG][HD]
  float* kn = qs + kMaxG * HD;  // [HD] new key (normalised, rotated)
  float* vn = kn + HD;          // [HD] new value
  float* sc = vn + HD;          // [kMaxG][64] scores, then weights
  float* st = sc + kMaxG * 64;  // [3][kMaxG]: m, l, rescale
  float* red = st + 4 * kMaxG;  // [KG][G][HD]
  float* kt = lds + attn_lds_head<HD>();  // [64][HD] key tile
  float* vt = kt + 64 * HD;               // [64][HD] value tile
  const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
  const int g = it.g, s0 = it.s0, s1 = it.s1;
  const bool has_new = s1 == P + 1;
  const float* cs = U(lp->rope) + (size_t)P * HD;
  const float inv = sqrtf((float)HD);
  const float vnew = has_new && tid < HD ? cload(U(lp->qkv) + U(lp->qd) + U(lp->kvd) + g * HD + tid) : 0.0f;
  const int nvec = G + (has_new ? 1 : 0);
  for (int v = wave; v < nvec; v += kW) {
    const bool key = v == G;
    const float* src = key ? U(lp->qkv) + U(lp->qd) + g * HD : U(lp->qkv) + (size_t)(g * G + v) * HD;
    norm_rope_vec<HD>(src, key ? ly.k_norm : ly.q_norm, U(lp->eps), cs, U(lp->pb), U(lp->po), U(lp->pst),
                      key ? kn : qs + v * HD);
  }
  if (has_new && tid < HD) vn[tid] = vnew;
  if (tid < kMaxG) {
    st[tid] = -INFINITY;
    st[kMaxG + tid] = 0.0f;
  }
  __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));  // first K/V tile in LDS
  __syncthreads();
  mark(2);
  const float* kb = ly.kcache + (size_t)g * U(lp->ctx) * HD;
  const float* vb = ly.vcache + (size_t)g * U(lp->ctx) * HD;
  // Scores: 8 lanes per key (KP dims each). P.V: thread (d, kg) takes the
  // tile's keys kg*KP .. kg*KP + KP - 1 (64 / KG = KP keys per group).
  const int d = tid % HD, kg = tid / HD, kk = tid / 8, pp = tid % 8;
  float acc[kMaxG];
#pragma unroll
  for (int h = 0; h < kMaxG; h++) acc[h] = 0.0f;
  for (int t0 = s0; t0 < s1; t0 += 64) {
    const int n = min(64, s1 - t0);
    if (t0 != s0) {  // later tiles (contexts over 64 keys per chunk)
      __syncthreads();  // previous tile fully read
      dma_kv_tile<HD>(kb, vb, t0, n, kt, vt);
      __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));
      __syncthreads();
    }
    if (has_new && P >= t0 && P < t0 + n) {  // row P: this step's key and value
      for (int e = tid; e < HD; e += kT) {
        kt[(P - t0) * HD + e] = kn[e];
        vt[(P - t0) * HD + e] = vn[e];
      }
      __syncthreads();
    }
    float kv[KP];
    lds_vec<KP>(kt + kk * HD + pp * KP, kv);
#pragma unroll
    for (int h = 0; h < kMaxG; h++) {
      if (h < G) {
        float q[KP];
        lds_vec<KP>(qs + h * HD + pp * KP, q);
        float a = 0.0f;
#pragma unroll
        for (int i = 0; i < KP; i++) a = fmaf(q[i], kv[i], a);
        a = group_sum<8>(a);
        if (pp == 0 && kk < n) sc[h * 64 + kk] = a / inv;
      }
    }
    __syncthreads();
    if (wave < G) {  // online softmax of head `wave` over this tile
      const float s = lane < n ? sc[wave * 64 + lane] : -INFINITY;
      const float mo = st[wave], mn = fmaxf(mo, wave_max(s));
      const float e = lane < n ? expf(s - mn) : 0.0f;
      sc[wave * 64 + lane] = e;  // 0 past the tile's keys
      const float sum = wave_sum(e);
      if (lane == 0) {
        const float f = expf(mo - mn);
        st[2 * kMaxG + wave] = f;
        st[kMaxG + wave] = st[kMaxG + wave] * f + sum;
        st[wave] = mn;
      }
    }
    __syncthreads();
    float v[KP];
#pragma unroll
    for (int i = 0; i < KP; i++) v[i] = kg * KP + i < n ? vt[(kg * KP + i) * HD + d] : 0.0f;
#pragma unroll
    for (int h = 0; h < kMaxG; h++) {
      if (h < G) {
        float w[KP];
        lds_vec<KP>(sc + h * 64 + kg * KP, w);
        float a = acc[h] * st[2 * kMaxG + h];
#pragma unroll
        for (int i = 0; i < KP; i++) a = fmaf(w[i], v[i], a);
        acc[h] = a;
      }
    }
  }
  mark(3);
#pragma unroll
  for (int h = 0; h < kMaxG; h++)
    if (h < G) red[(kg * G + h) * HD + d] = acc[h];
  __syncthreads();
  for (int o = tid; o < G * HD; o += kT) {
    const int h = o / HD, dd = o % HD;
    float a = 0.0f;
    for (int k = 0; k < KG; k++) a += red[(k * G + h) * HD + dd];
    float* pp2 = U(lp->part) + ((size_t)(g * G + h) * U(lp->max_chunks) + it.c) * (HD + 2);
    cstore(pp2 + 2 + dd, a);
    if (dd == 0) {
      cstore(pp2, st[h]);
      cstore(pp2 + 1, st[kMaxG + h]);
    }
  }
  if (has_new) {  // cache row P of kv head g, read by later steps
    float* kc = ly.kcache + ((size_t)g * U(lp->ctx) + P) * HD;
    float* vc = ly.vcache + ((size_t)g * U(lp->ctx) + P) * HD;
    for (int e = tid; e < HD; e += kT) {
      gstore(kc + e, kn[e]);
      gstore(vc + e, vn[e]);
    }
  }
  mark(4);
}

// att[o] for o in [o0, o0 + n): M = max_c m_c, w_c = e^(m_c - M),
// att = sum_c w_c acc_c / sum_c w_c l_c.
template <int HD, typename Mark>
__device__ __forceinline__ void combine_phase(const DecodeParams* lp, int P, float* lds, int worker,
                                              int workers, Mark mark) {
  const int opb = U(lp->comb_outputs);
  float* wts = lds;       // [64]
  float* red = lds + 72;  // [nch][opb]
  int nch, len;
  attn_chunks(P + 1, U(lp->max_chunks), nch, len);
  for (int o0 = worker * opb; o0 < U(lp->qd); o0 += workers * opb) {
    const int h = o0 / HD, d0 = o0 % HD;
    const float* pb = U(lp->part) + (size_t)h * U(lp->max_chunks) * (HD + 2);
    const int c = threadIdx.x / opb, dd = threadIdx.x % opb;
    const float v = c < nch ? cload(pb + (size_t)c * (HD + 2) + 2 + d0 + dd) : 0.0f;
    if (threadIdx.x == 0) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      mark(3);
    }
    if (threadIdx.x < WAVE) {
      const int i = threadIdx.x;
      const float m = i < nch ? cload(pb + (size_t)i * (HD + 2)) : -INFINITY;
      const float l = i < nch ? cload(pb + (size_t)i * (HD + 2) + 1) : 0.0f;
      const float M = wave_max(m);
      const float w = i < nch ? expf(m - M) : 0.0f;
      const float L = wave_sum(w * l);
      wts[i] = w;
      if (i == 0) wts[64] = L;
    }
    __syncthreads();
    mark(2);
    if (c < nch) red[c * opb + dd] = wts[c] * v;
    __syncthreads();
    if ((int)threadIdx.x < opb) {
      float o = 0.0f;
      for (int k = 0; k < nch; k++) o += red[k * opb + threadIdx.x];
      cstore(U(lp->att) + o0 + threadIdx.x, o / wts[64]);
    }
    __syncthreads();
  }
  mark(4);
}

// -------------------------------------------------------------- argmax --

__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
  // Larger value wins; equal values keep the lower index. NaN never wins.
  return v > bv || (v == bv && i < bi);
}

__device__ __forceinline__ void block_best(float& bv, int& bi, float* sv, int* si) {
  __syncthreads();
  sv[threadIdx.x] = bv;
  si[threadIdx.x] = bi;
  __syncthreads();
  for (int st = kT / 2; st > 0; st >>= 1) {
    if ((int)threadIdx.x < st &&
        better(sv[threadIdx.x + st], si[threadIdx.x + st], sv[threadIdx.x], si[threadIdx.x])) {
      sv[threadIdx.x] = sv[threadIdx.x + st];
      si[threadIdx.x] = si[threadIdx.x + st];
    }
    __syncthreads();
  }
  bv = sv[0];
  bi = si[0];
}

// ---------------------------------------------------------------- step --

// Phase tracer, on the first worker (block 1) when enabled: time before
// each barrier (work, row 0), inside it (wait, row 1), and for the phase
// after it the end of input staging (row 2), weight loop (3) and epilogue
// (4). Accumulated in LDS (no global memory traffic of its own between
// barriers) and added to the global trace at the end of the launch.
struct Tracer {
  unsigned long long* acc;  // LDS, block 1 only; null: off
  int k, nbar;
  uint64_t last;
};

__device__ __forceinline__ void mark(const Tracer& tr, int which) {
  if (tr.acc && threadIdx.x == 0 && tr.k > 0)
    tr.acc[which * tr.nbar + tr.k - 1] += wall_clock64() - tr.last;
}

// Worker side of a phase boundary: arrive, issue the next phase's loads
// (`prefetch`), wait.
template <typename F>
__device__ __forceinline__ void phase_boundary(GridSync& g, Tracer& tr, F prefetch) {
  const bool on = tr.acc && threadIdx.x == 0;
  uint64_t t0 = 0;
  if (on) t0 = wall_clock64();
  grid_arrive(g);
  prefetch();
  grid_wait(g);
  if (on) {
    const uint64_t t1 = wall_clock64();
    tr.acc[tr.k] += t0 - tr.last;
    tr.acc[tr.nbar + tr.k] += t1 - t0;
    tr.last = t1;
  }
  tr.k++;
}

// Layer descriptor l, copied through a global pointer (scalar loads).
__device__ __forceinline__ DecodeLayer layer_at(const DecodeParams* lp, int l) {
  DecodeLayer ly;
  static_assert(sizeof(DecodeLayer) % 8 == 0, "pointer-sized fields");
  const __attribute__((address_space(1))) uint64_t* src =
      (const __attribute__((address_space(1))) uint64_t*)(U(lp->layers) + l);
  uint64_t* dst = (uint64_t*)&ly;
#pragma unroll
  for (int i = 0; i < (int)(sizeof(DecodeLayer) / 8); i++) dst[i] = src[i];
  return ly;
}

// Phases of a step: 6 per layer (QKV, attention, combine, O, gate/up,
// down), then the logits.
enum PhaseKind { PH_QKV, PH_ATTN, PH_COMB, PH_O, PH_GU, PH_DOWN, PH_LOGITS };

__device__ __forceinline__ int phase_kind(int ph, int L) { return ph == 6 * L ? PH_LOGITS : ph % 6; }

// What a GEMV phase multiplies, with what input and epilogue.
struct GemvPhase {
  const uint16_t *w, *w2;
  int N, K;
  DecodeGemvPlan plan;
  int epi;
  const float* src;      // input row (agent-coherent), unless emb
  const uint16_t* emb;   // embedding row (layer 0 QKV), or null
  const uint16_t* nw;    // RMSNorm weight of the input, or null
};

__device__ __forceinline__ GemvPhase gemv_phase(const DecodeParams* lp, int ph, int tok) {
  GemvPhase g;
  g.w2 = nullptr;
  g.emb = nullptr;
  g.nw = nullptr;
  const int kind = phase_kind(ph, U(lp->L));
  if (kind == PH_LOGITS) {
    g.w = U(lp->out_w);
    g.N = U(lp->V);
    g.K = U(lp->d);
    g.plan = U(lp->p_logits);
    g.epi = EPI_LOGITS;
    g.src = U(lp->x);
    g.nw = U(lp->out_norm);
    return g;
  }
  const int l = ph / 6;
  const DecodeLayer ly = layer_at(lp, l);
  if (kind == PH_QKV) {
    g.w = ly.qkv;
    g.N = U(lp->qkv_rows);
    g.K = U(lp->d);
    g.plan = U(lp->p_qkv);
    g.epi = EPI_QKV;
    g.src = U(lp->x);
    if (l == 0) g.emb = U(lp->emb) + (size_t)tok * U(lp->d);
    g.nw = ly.attn_norm;
  } else if (kind == PH_O) {
    g.w = ly.o;
    g.N = U(lp->d);
    g.K = U(lp->qd);
    g.plan = U(lp->p_o);
    g.epi = EPI_RESIDUAL;
    g.src = U(lp->att);
  } else if (kind == PH_GU) {
    g.w = ly.gate;
    g.w2 = ly.up;
    g.N = U(lp->H);
    g.K = U(lp->d);
    g.plan = U(lp->p_gu);
    g.epi = EPI_SWIGLU;
    g.src = U(lp->x);
    g.nw = ly.ffn_norm;
  } else {  // PH_DOWN
    g.w = ly.down;
    g.N = U(lp->d);
    g.K = U(lp->H);
    g.plan = U(lp->p_down);
    g.epi = EPI_RESIDUAL;
    g.src = U(lp->act);
  }
  return g;
}

// The parameters are read from device memory (not kernel arguments): the
// barriers' memory clobbers make the compiler reload them per phase instead
// of keeping dozens of them live in scalar registers for the whole step.
template <int HD>
__global__ __launch_bounds__(kT, 1) void decode_step_kernel(const DecodeParams* params) {
  extern __shared__ __attribute__((aligned(16))) float lds_all[];
  {
    const unsigned* src = (const unsigned*)params;
    for (int i = threadIdx.x; i < (int)(sizeof(DecodeParams) / 4); i += kT)
      ((unsigned*)lds_all)[i] = src[i];
    __syncthreads();
  }
  const DecodeParams* lp = (const DecodeParams*)lds_all;
  float* lds = lds_all + kParamFloats;
  const int kmax = max(U(lp->d), max(U(lp->qd), U(lp->H)));
  float* xs = lds;
  float* part1 = lds + kmax;
  float* part2 = part1 + kDecodePartMax;
  float* red = part2 + kDecodePartMax;  // [64]

  GridSync g{U(lp->sync_state), U(lp->sync_err), (unsigned)cload((const int*)U(lp->epoch)) + 1u};
  const int P = cload(U(lp->pos)), tok = cload(U(lp->tok));
  const int nbar = decode_barriers(U(lp->L));

  if (blockIdx.x == 0) {
    // Master: coordinates every barrier, then reduces the workers' argmax.
    for (int k = 0; k < nbar; k++) grid_master(g);
    float bv = -INFINITY;
    int bi = U(lp->V);
    for (int b = threadIdx.x; b < (int)gridDim.x - 1; b += kT) {
      const float v = cload(U(lp->am_v) + b);
      const int i = cload(U(lp->am_i) + b);
      if (better(v, i, bv, bi)) {
        bv = v;
        bi = i;
      }
    }
    block_best(bv, bi, part1, (int*)part2);
    if (threadIdx.x == 0) {
      // Sequential-scan semantics: a NaN at index 0 is never replaced, and
      // when nothing compares greater than element 0 the answer is 0.
      const float x0 = cload(U(lp->am_v) + gridDim.x - 1);  // logits[0]
      int best = bi;
      if (best >= U(lp->V) || x0 != x0) best = 0;
      *U(lp->next) = best;
      if (U(lp->seq)) {
        const int k = *U(lp->seq_len);
        U(lp->seq)[k] = best;
        *U(lp->seq_len) = k + 1;
      }
      *U(lp->pos) = P + 1;
      *U(lp->epoch) = g.seq - 1;
    }
    return;
  }

  const int w = blockIdx.x - 1, NW = gridDim.x - 1;
  Tracer tr{nullptr, 0, nbar, 0};
  if (U(lp->trace) && w == 0) {
    tr.acc = (unsigned long long*)((char*)lds + U(lp->trace_lds));
    for (int i = threadIdx.x; i < kDecodeTraceRows * nbar; i += kT) tr.acc[i] = 0;
    __syncthreads();
    tr.last = wall_clock64();
  }
  auto mk = [&](int which) { mark(tr, which); };
  const int last = 6 * U(lp->L);  // the logits phase

  Batch cur;
  Cursor ld{0, 0, 0};
  Job job;
  {
    const GemvPhase gp = gemv_phase(lp, 0, tok);
    job = make_job(gp.w, gp.w2, gp.N, gp.K, gp.plan, w);
    load_batch(job, ld, cur);
  }
  for (int ph = 0;; ph++) {
    const int kind = phase_kind(ph, U(lp->L));
    if (kind == PH_ATTN) {
      attention_phase<HD>(lp, layer_at(lp, ph / 6), P, attn_item(lp, P, w), lds, mk);
    } else if (kind == PH_COMB) {
      combine_phase<HD>(lp, P, lds, w, NW, mk);
    } else {
      const GemvPhase gp = gemv_phase(lp, ph, tok);
      // hidden-state capture: x entering layer l (l > 0) is layer l-1's
      // output; x entering the logits is the last layer's
      float *cap_raw = nullptr, *cap_norm = nullptr;
      if (U(lp->cap) && w == 0 && (kind == PH_QKV || kind == PH_LOGITS) && ph > 0) {
        cap_raw = U(lp->cap) + (size_t)(ph / 6 - 1) * U(lp->d);
        if (kind == PH_LOGITS) cap_norm = U(lp->cap_final);
      }
      stage_input(gp.src, gp.emb, U(lp->x), gp.K, gp.nw, U(lp->eps), xs, red, w, NW, cap_raw, cap_norm);
      mk(2);
      gemv_run(job, cur, ld, xs, part1, part2, mk);
      // dead until the next prefetch (frees their registers meanwhile)
      cur = Batch{};
      ld = Cursor{0, 0, 0};
      float bv = -INFINITY;
      int bi = U(lp->V);
      for (int r = threadIdx.x; r < job.rows; r += kT) {
        const int row = job.row0 + r;
        const float y = part1[r];
        switch (gp.epi) {
          case EPI_QKV: cstore(U(lp->qkv) + row, y); break;
          case EPI_RESIDUAL: cstore(U(lp->x) + row, cload(U(lp->x) + row) + y); break;
          case EPI_SWIGLU: cstore(U(lp->act) + row, silu_mul(y, part2[r])); break;
          default:  // EPI_LOGITS
            if (U(lp->logits)) U(lp->logits)[row] = y;
            if (row == 0) cstore(U(lp->am_v) + NW, y);  // logits[0] for the NaN rule
            if (better(y, row, bv, bi)) {
              bv = y;
              bi = row;
            }
        }
      }
      if (gp.epi == EPI_LOGITS) {
        block_best(bv, bi, part1, (int*)part2);
        if (threadIdx.x == 0) {
          cstore(U(lp->am_v) + w, bv);
          cstore(U(lp->am_i) + w, bi);
        }
      }
      mk(4);
      job = Job{};
      // Keep the epilogue's stores ahead of the next phase's weight loads.
      asm volatile("" ::: "memory");
    }
    if (ph == last) break;
    const int nx = ph + 1, nkind = phase_kind(nx, U(lp->L));
    phase_boundary(g, tr, [&] {
      if (nkind == PH_ATTN) {
        // the item's first K/V tile (rows of earlier steps) goes to LDS
        const AttnItem item = attn_item(lp, P, w);
        if (item.valid) {
          const DecodeLayer ly = layer_at(lp, nx / 6);
          float* kt = lds + attn_lds_head<HD>();
          dma_kv_tile<HD>(ly.kcache + (size_t)item.g * U(lp->ctx) * HD,
                          ly.vcache + (size_t)item.g * U(lp->ctx) * HD, item.s0,
                          min(64, item.s1 - item.s0), kt, kt + 64 * HD);
        }
      } else if (nkind != PH_COMB) {
        const GemvPhase np = gemv_phase(lp, nx, tok);
        job = make_job(np.w, np.w2, np.N, np.K, np.plan, w);
        ld = Cursor{0, 0, 0};
        load_batch(job, ld, cur);
      }
    });
  }
  phase_boundary(g, tr, [] {});
  if (tr.acc) {
    __syncthreads();
    for (int i = threadIdx.x; i < kDecodeTraceRows * nbar; i += kT) U(lp->trace)[i] += tr.acc[i];
  }
}

template <int HD>
void launch(const DecodeParams& p, const DecodeParams* dp, int blocks, hipStream_t s) {
  const void* fn = (const void*)decode_step_kernel<HD>;
  const size_t lds = kParamFloats * sizeof(float) +
                     (p.trace ? p.trace_lds + decode_trace_lds_bytes(p.L) : decode_lds_bytes(p));
  static size_t attr_lds = 0;  // largest dynamic LDS size enabled so far
  if (lds > attr_lds) {
    HIP_CHECK(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
    attr_lds = lds;
  }
  const DecodeParams* arg = dp;
  void* args[] = {&arg};
  HIP_CHECK(hipLaunchCooperativeKernel(fn, dim3(blocks), dim3(kT), args, lds, s));
}

}  // namespace

DecodeGemvPlan decode_gemv_plan(int N, int K, int blocks) {
  const int rb = (N + blocks - 1) / blocks;
  const int chunks = (K + 7) / 8;
  DecodeGemvPlan best{rb, 1, chunks};
  long best_cost = -1;
  for (int S = 1; S <= 16; S *= 2) {
    if (rb * S > kDecodePartMax) break;
    const int ks = (chunks + S - 1) / S;
    const long it = (ks + WAVE - 1) / WAVE;
    const long per_wave = (rb * S + kW - 1) / kW;
    // items of the busiest wave; a reduction per slice costs about an item
    const long cost = per_wave * (it + 1);
    if (best_cost < 0 || cost < best_cost) {
      best_cost = cost;
      best = DecodeGemvPlan{rb, S, ks};
    }
  }
  return best;
}

size_t decode_trace_lds_bytes(int L) {
  return (size_t)kDecodeTraceRows * decode_barriers(L) * sizeof(unsigned long long);
}

size_t decode_lds_bytes(const DecodeParams& p) {
  const size_t kmax = std::max(p.d, std::max(p.qd, p.H));
  const size_t gemv = (kmax + 2 * kDecodePartMax + 128) * sizeof(float);
  const size_t attn = ((size_t)10 * p.hd + kMaxG * 64 + 4 * kMaxG + (size_t)kT * kMaxG +
                       128 * (size_t)p.hd) * sizeof(float);  // attn_lds_head + K/V tiles
  const size_t comb = (72 + (size_t)kT) * sizeof(float);
  return std::max(kMinLds, std::max(gemv, std::max(attn, comb)));
}

bool decode_supported(int d, int H, int qh, int kvh, int hd, int qd, int V, int blocks,
                      size_t lds_limit) {
  if (hd != 16 && hd != 32 && hd != 64 && hd != 128) return false;
  const int workers = blocks - 1;
  if (kvh <= 0 || qh % kvh || qh / kvh > kMaxG || kvh > workers) return false;
  if (d % 8 || H % 8 || qd % 8 || d < 8) return false;
  if ((V + workers - 1) / workers > kDecodePartMax) return false;
  DecodeParams p{};
  p.d = d;
  p.H = H;
  p.qd = qd;
  p.hd = hd;
  return decode_lds_bytes(p) <= lds_limit;
}

int decode_blocks() {
  int dev, cus;
  HIP_CHECK(hipGetDevice(&dev));
  HIP_CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev));
  return cus;
}

void decode_step(const DecodeParams& p, const DecodeParams* dp, int blocks, hipStream_t s) {
  if (blocks <= 0 || blocks > kSyncMaxBlocks) ST_DIE("decode step: bad block count");
  if (blocks < 2) ST_DIE("decode step needs a master and at least one worker block");
  if (p.max_chunks <= 0 || p.max_chunks > WAVE || p.max_chunks * p.kvh > blocks - 1)
    ST_DIE("decode step: bad attention chunking");
  if (p.comb_outputs <= 0 || p.hd % p.comb_outputs || p.comb_outputs * p.max_chunks > kT)
    ST_DIE("decode step: bad combine split");
  switch (p.hd) {
    case 16: launch<16>(p, dp, blocks, s); break;
    case 32: launch<32>(p, dp, blocks, s); break;
    case 64: launch<64>(p, dp, blocks, s); break;
    case 128: launch<128>(p, dp, blocks, s); break;
    default: ST_DIE("decode step supports head_dim 16, 32, 64 or 128");
  }
}

}  // namespace sg
