// Persistent decode step on gfx950: one launch per generated token of a
// dense model (reference transformer_predict with one token,
// source/transformer.c:1186-1602, then the greedy argmax of
// source/sampler.c).
//
// The grid is one 768-thread block per compute unit, all resident at once
// (cooperative launch). Block 0 only coordinates the grid barriers
// (grid_sync.h) and reduces the argmax; the other blocks are workers. The
// step is a sequence of phases separated by grid barriers:
//
//   per layer: QKV GEMV (RMSNorm prologue; layer 0 embeds the token)
//              attention over (kv head, key chunk) items, QK-norm + RoPE,
//                the last item of each kv head combining the chunks;
//                writes the new key/value row into the cache
//              O GEMV + residual
//              gate/up GEMV + SwiGLU (RMSNorm prologue)
//              down GEMV + residual
//   then:      logits GEMV (final RMSNorm prologue) + per-block argmax
//              argmax of the block winners, *next, seq, *pos += 1
//
// Roles inside a worker block. Waves 0-7 (stream waves) only load weights:
// each GEMV phase gives the worker `rb` consecutive output rows cut into S
// slices per row; the stream waves take slices round-robin and walk them
// with 128-bit non-temporal loads (8 bf16 per lane), three batches of 8
// loads per lane in rotation (two in flight while one is multiplied). As
// soon as a stream wave has multiplied its last batch it issues the first
// two batches of the next GEMV phase, so the weight stream continues through
// the epilogue, the grid barrier, the input staging and (after QKV) the
// whole attention phase. Waves 8-11 (control waves) do everything else:
// coherent loads of the input row, RMSNorm, slice-sum reduction and
// epilogue stores, barrier arrival and polling, attention. Their memory
// operations never queue behind weight loads (vector memory operations of
// a wave complete in issue order, but each wave has its own queue), and the
// block barriers let stream waves keep their loads in flight.
//
// Activations crossing blocks (x, q/k/v, attention partials and outputs,
// SwiGLU output, argmax winners) are written and read with agent-coherent
// accesses only; the barriers carry no cache fences. The residual rows a
// worker updates are kept in LDS from the staging of the same vector, so
// the residual epilogues store without loading.
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

constexpr int kS = 512;             // stream threads (waves 0-7)
constexpr int kC = 256;             // control threads (waves 8-11)
constexpr int kT = kS + kC;         // block size
constexpr int kW = kS / WAVE;       // stream waves
constexpr int kCW = kC / WAVE;      // control waves
constexpr int kU = 8;               // weight loads per lane per batch (4 per matrix for a pair)
constexpr int kMaxG = 8;            // q heads per kv head
constexpr int kMinChunk = 16;       // keys per attention item, at least
constexpr int kTile = 32;           // keys per attention LDS tile
constexpr int kMaxChunks = 32;      // key chunks per kv head
constexpr int kOwnMax = 256;        // residual rows per worker kept in LDS
constexpr int kStageB = 12;         // 64-bit coherent loads per control thread per round
constexpr int kNormPairs = 16;      // norm-weight pairs per control thread held in registers
constexpr int kCtl = 72;            // LDS floats: block reduction slots and flags
constexpr size_t kMinLds = 81 * 1024;  // more than half of a CU's LDS
static_assert(kT == kDecodeThreads, "block size");

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

__device__ __forceinline__ bool control_wave() { return threadIdx.x >= kS; }

// Block barrier of all 12 waves. With VM, control waves first wait for
// their vector memory operations (their loads and stores complete); stream
// waves never wait for theirs (weight loads stay in flight). LDS operations
// of every wave complete before the barrier. The empty asm statements keep
// the compiler from moving memory accesses across it.
template <bool VM>
__device__ __forceinline__ void bar() {
  asm volatile("" ::: "memory");
  if (VM && control_wave())
    __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));
  else
    __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(63));
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Worker side of a grid barrier (the master runs grid_master): arrival
// once the control waves' stores are complete, then the wait.
// Barrier of the four control waves only (stream waves never take part, so
// a stream wave stalled issuing loads delays nobody): each control wave
// adds 1 to an LDS counter and waits for the count of the barrier; with
// VM it first waits for its own vector memory operations. Bounded: after
// twice the grid-barrier time-out it records the error and goes on.
struct CSync {
  unsigned* ctr;  // LDS arrival counter, 0 at kernel start
  unsigned n;     // arrivals that complete the next barrier, minus kCW
  unsigned* err;  // the grid's error flag
};

template <bool VM>
__device__ __forceinline__ void csync(CSync& cs) {
  asm volatile("" ::: "memory");
  if (VM)
    __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(0));
  else
    __builtin_amdgcn_s_waitcnt(waitcnt_vm_lgkm0(63));
  cs.n += kCW;
  if (threadIdx.x % WAVE == 0)
    __hip_atomic_fetch_add(cs.ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  const uint64_t t0 = wall_clock64();
  while ((int)(U(__hip_atomic_load(cs.ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) - cs.n) < 0) {
    __builtin_amdgcn_s_sleep(1);
    if (wall_clock64() - t0 > 2 * kSyncTimeoutTicks) {
      if (threadIdx.x % WAVE == 0) sync_store(cs.err, 1u);
      break;
    }
  }
  asm volatile("" ::: "memory");
}

// Worker side of a grid barrier (the master runs grid_master), by the
// control waves: arrival once their stores are complete, then the wait.
__device__ __forceinline__ void worker_arrive(const GridSync& g, CSync& cs) {
  csync<true>(cs);
  if (threadIdx.x == kS) sync_store(g.state + kSyncSlotWords * (1 + blockIdx.x), g.seq);
}

__device__ __forceinline__ void worker_wait(GridSync& g, CSync& cs) {
  if (threadIdx.x == kS) sync_wait(g.state, g.seq, g.err);
  csync<false>(cs);
  g.seq++;
}

// ---------------------------------------------------------------- GEMV --
//
// One code path serves every GEMV phase (the kernel is large, and one copy
// of its streaming loop stays in the instruction cache): the matrix pair of
// gate/up (`dual`), the epilogue and the input staging are run-time
// choices. Only stream waves run the Job / Batch code.

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

__device__ __forceinline__ int job_batches(const Job& j) {
  const int per = j.w2 ? kU / 2 : kU;
  return (j.items + per - 1) / per;
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

// Issues exactly kU loads: kU items of one matrix, or kU/2 items of each
// matrix of a pair (slots kU/2 + u hold the second matrix's item u). Slots
// past the wave's work load `safe` (lines already in flight). Straight-line
// code: the per-lane and per-wave conditions are selects.
template <bool DUAL>
__device__ __forceinline__ void load_batch(const Job& j, Cursor& c, Batch& B) {
  constexpr int per = DUAL ? kU / 2 : kU;
  const int lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
#pragma unroll
  for (int u = 0; u < per; u++) {
    const unsigned off = c.n < j.items ? item_offset(j, c, lane, wave) : j.safe;
    B.a[u] = load_nt_u4(j.w + off);
    if (DUAL) B.a[u + per] = load_nt_u4(j.w2 + off);
  }
}

// Multiplies a batch into the running slice sums; at each slice end the
// wave's sums go to part1[q] (part2[q]) at the block slice index q. Lanes
// past their slice (and items past the wave's work) keep their sums: the
// products are computed for every lane and selected, so the only branches
// are the wave-uniform slice ends.
template <bool DUAL>
__device__ __forceinline__ void mul_batch(const Job& j, Cursor& c, const Batch& B, const float* xs,
                                          float& acc, float& acc2, float* part1, float* part2) {
  constexpr int per = DUAL ? kU / 2 : kU;
  const int lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
#pragma unroll
  for (int u = 0; u < per; u++) {
    const bool live = c.n < j.items;
    const int q = wave + kW * c.sl;
    const int part = q & ((1 << j.log2s) - 1);
    const int ch = c.i * WAVE + lane, col = (part * j.ks + ch) * 8;
    const bool ok = live && ch < j.ks && col < j.K;
    const int cx = ok ? col : 0;
    const float4 x0 = *(const float4*)(xs + cx);
    const float4 x1 = *(const float4*)(xs + cx + 4);
    const float a1 = dot8(B.a[u], x0, x1, acc);
    acc = ok ? a1 : acc;
    if (DUAL) {
      const float a2 = dot8(B.a[u + per], x0, x1, acc2);
      acc2 = ok ? a2 : acc2;
    }
    if (live) {
      c.n++;
      if (++c.i == j.it) {  // slice done
        const float s1 = wave_total(acc);
        if (lane == 0) part1[q] = s1;
        if (DUAL) {
          const float s2 = wave_total(acc2);
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

// First two batches of a job (the loader cursor `ld` moves past them).
template <bool DUAL>
__device__ __forceinline__ void gemv_prefetch(const Job& j, Cursor& ld, Batch& b0, Batch& b1) {
  load_batch<DUAL>(j, ld, b0);
  load_batch<DUAL>(j, ld, b1);
}

__device__ __forceinline__ void gemv_prefetch_any(const Job& j, Cursor& ld, Batch& b0, Batch& b1) {
  if (j.w2)
    gemv_prefetch<true>(j, ld, b0, b1);
  else
    gemv_prefetch<false>(j, ld, b0, b1);
}

// A GEMV phase on a stream wave, batches 0 and 1 already in flight in b0
// and b1, the input row in LDS xs: slice sums go to part1 (part2 for the
// second matrix of a pair) at the block slice index. The two batch buffers
// alternate without copies (a register copy would wait for the loads that
// fill it): batch b+2 is issued as soon as batch b is multiplied, so batch
// b+1 is in flight while b is multiplied.
template <bool DUAL>
__device__ __forceinline__ void gemv_run(const Job& j, Batch& b0, Batch& b1, Cursor ld,
                                         const float* xs, float* part1, float* part2) {
  const int nb = job_batches(j);
  Cursor cc{0, 0, 0};
  float acc = 0.0f, acc2 = 0.0f;
  for (int b = 0; b < nb; b += 2) {
    mul_batch<DUAL>(j, cc, b0, xs, acc, acc2, part1, part2);
    if (b + 2 < nb) load_batch<DUAL>(j, ld, b0);
    if (b + 1 >= nb) break;
    mul_batch<DUAL>(j, cc, b1, xs, acc, acc2, part1, part2);
    if (b + 3 < nb) load_batch<DUAL>(j, ld, b1);
  }
}

// Input row of a GEMV phase into LDS xs[0, K), by the control waves
// (ends with the block barrier that releases the stream waves):
//   emb != null: x = embedding row emb (bf16 -> fp32, exact);
//   otherwise:   x = src read agent-coherent, kStageB 64-bit loads per
//                thread in flight before any is used;
// then, when nw != null, xs = RMSNorm(x) with weight nw, else xs = x.
// x[own0, own0 + nown) (before the norm) is also kept in xown.
// cap_raw / cap_norm (null, or chosen by the caller): copies of x before and
// after the RMSNorm. Each control thread handles the pairs
// ct, ct + kC, ... throughout, so only the norm's sum needs a barrier.
__device__ __forceinline__ void stage_input(const float* src, const uint16_t* emb, int K,
                                            const uint16_t* nw, float eps, float* xs, float* red,
                                            float* xown, int own0, int nown, float* cap_raw,
                                            float* cap_norm, CSync& cs) {
  constexpr bool CTRL = true;
  const int ct = threadIdx.x - kS, pairs = K / 2;
  float ss = 0.0f;
  auto put = [&](int idx, float a, float b) {
    *(float2*)(xs + 2 * idx) = make_float2(a, b);
    ss = fmaf(a, a, ss);
    ss = fmaf(b, b, ss);
    const int k0 = 2 * idx - own0;
    if ((unsigned)k0 < (unsigned)nown) xown[k0] = a;
    if ((unsigned)(k0 + 1) < (unsigned)nown) xown[k0 + 1] = b;
    if (cap_raw) {
      gstore(cap_raw + 2 * idx, a);
      gstore(cap_raw + 2 * idx + 1, b);
    }
  };
  // norm weights of the thread's first kNormPairs pairs, loaded with the
  // input (one memory round trip for both)
  uint32_t nwp[kNormPairs];
  if constexpr (CTRL) {
    if (nw) {
#pragma unroll
      for (int r = 0; r < kNormPairs; r++) {
        const int idx = min(ct + r * kC, pairs - 1);
        nwp[r] = *(const __attribute__((address_space(1))) uint32_t*)(nw + 2 * idx);
      }
    }
    if (emb) {
      for (int base = ct; base < pairs; base += kC * kNormPairs) {
        uint32_t e[kNormPairs];
#pragma unroll
        for (int i = 0; i < kNormPairs; i++)
          e[i] = *(const __attribute__((address_space(1))) uint32_t*)(emb + 2 * min(base + i * kC, pairs - 1));
#pragma unroll
        for (int i = 0; i < kNormPairs; i++)
          if (base + i * kC < pairs) put(base + i * kC, bf16_lo(e[i]), bf16_hi(e[i]));
      }
    } else {
      const unsigned long long* s2 = (const unsigned long long*)src;
      for (int base = ct; base < pairs; base += kC * kStageB) {
        unsigned long long v[kStageB];
#pragma unroll
        for (int i = 0; i < kStageB; i++) {
          const int idx = base + i * kC;
          v[i] = idx < pairs ? __hip_atomic_load((const __attribute__((address_space(1))) unsigned long long*)(s2 + idx),
                                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                             : 0ull;
        }
#pragma unroll
        for (int i = 0; i < kStageB; i++) {
          const int idx = base + i * kC;
          if (idx < pairs) put(idx, __uint_as_float((unsigned)v[i]), __uint_as_float((unsigned)(v[i] >> 32)));
        }
      }
    }
  }
  if (nw) {
    if constexpr (CTRL) {
      ss = wave_sum(ss);
      if (threadIdx.x % WAVE == 0) red[ct / WAVE] = ss;
    }
    csync<false>(cs);
    if constexpr (CTRL) {
      float tot = 0.0f;
#pragma unroll
      for (int i = 0; i < kCW; i++) tot += red[i];
      const float s = rms_scale(tot, K, eps);
      auto apply = [&](int idx, uint32_t wp) {
        float2 v = *(float2*)(xs + 2 * idx);
        v.x = (v.x * s) * bf16_lo(wp);
        v.y = (v.y * s) * bf16_hi(wp);
        *(float2*)(xs + 2 * idx) = v;
        if (cap_norm) {
          gstore(cap_norm + 2 * idx, v.x);
          gstore(cap_norm + 2 * idx + 1, v.y);
        }
      };
#pragma unroll
      for (int r = 0; r < kNormPairs; r++)
        if (ct + r * kC < pairs) apply(ct + r * kC, nwp[r]);
      for (int idx = ct + kNormPairs * kC; idx < pairs; idx += kC)
        apply(idx, *(const __attribute__((address_space(1))) uint32_t*)(nw + 2 * idx));
    }
  }
  bar<false>();  // xs ready: the stream waves start
}

// ----------------------------------------------------------- attention --

__device__ __forceinline__ void attn_chunks(int total, int max_chunks, int& nch, int& len) {
  nch = min(max_chunks, (total + kMinChunk - 1) / kMinChunk);
  len = (total + nch - 1) / nch;
  nch = (total + len - 1) / len;  // no empty chunk
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

// LDS layout of the attention phase (floats, from the start of the region
// shared with the GEMV input row and slice sums).
template <int HD>
struct AttLds {
  static constexpr int qs = 0;                       // [kMaxG][HD]
  static constexpr int kn = qs + kMaxG * HD;         // [HD] new key
  static constexpr int vn = kn + HD;                 // [HD] new value
  static constexpr int sc = vn + HD;                 // [kMaxG][kTile]
  static constexpr int st = sc + kMaxG * kTile;      // [3][kMaxG] m, l, rescale
  static constexpr int wts = st + 4 * kMaxG;         // [kMaxG][kMaxChunks + 1]
  static constexpr int tiles = wts + kMaxG * (kMaxChunks + 1) + 4;  // [2][K|V][kTile][HD]
  static constexpr int total = tiles + 4 * kTile * HD;
  static_assert(tiles % 4 == 0, "16-byte aligned tiles");
};

// Keys [t0, t0 + n) of a kv head (rows of HD floats, contiguous) into the
// LDS tiles kt / vt by the global-to-LDS DMA of the control waves: 16
// bytes per lane, each wave filling 1 KiB of LDS per instruction, no
// registers held.
template <int HD>
__device__ __forceinline__ void dma_kv(const float* kb, const float* vb, int t0, int n, float* kt,
                                       float* vt) {
  const int units = n * HD / 4;
  const int ct = threadIdx.x - kS, wave = ct / WAVE, lane = ct % WAVE;
  const float* ks = kb + (size_t)t0 * HD;
  const float* vs = vb + (size_t)t0 * HD;
  for (int u0 = wave * WAVE; u0 < units; u0 += kC) {
    const int u = u0 + lane;
    if (u < units) {
      __builtin_amdgcn_global_load_lds((const void*)(ks + u * 4), (lds_ptr)(kt + u0 * 4), 16, 0, 0);
      __builtin_amdgcn_global_load_lds((const void*)(vs + u * 4), (lds_ptr)(vt + u0 * 4), 16, 0, 0);
    }
  }
}

// Attention work item of a worker: kv head g, key chunk c = [s0, s1) of
// nch chunks.
struct AttnItem {
  bool valid;
  int g, c, s0, s1, nch;
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
  it.nch = nch;
  return it;
}

// RMSNorm (when norm) and RoPE of one head vector held by a control wave:
// xv / wv are the lane's elements lane + i*64 of the vector and of the norm
// weights, fr / fi the rotation of the lane's pair (elements lane*pst and
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

// Attention item of this worker, by the control waves: for the G query heads of kv head g, the
// softmax statistics (max m, sum l) and the unnormalised P.V over the
// item's keys, in tiles of kTile keys (the first put in flight to LDS
// before the barrier that precedes this phase, later ones double-buffered),
// with an online rescale; row P, written by this step, comes from the new
// key and value. The partials are stored agent-coherent and the worker
// counts itself on the kv head's counter; the last worker of the head
// combines all chunks:
//   att = sum_c e^(m_c - M) o_c / sum_c e^(m_c - M) l_c,  M = max_c m_c.
// Stage loads are issued before any is used (one memory round trip each).
template <int HD, typename Mark>
__device__ __forceinline__ void attention_phase(const DecodeParams* lp, const DecodeLayer& ly, int P,
                                                const AttnItem& it, float* la, int* flag, CSync& cs,
                                                Mark mark) {
  constexpr bool CTRL = true;
  using A = AttLds<HD>;
  constexpr int KP = HD / 8;                           // dims per lane for scores
  constexpr int OPT = (kMaxG * HD + kC - 1) / kC;      // P.V outputs per control thread
  constexpr int PER = (HD + WAVE - 1) / WAVE;
  constexpr int MAXV = (kMaxG + 1 + kCW - 1) / kCW;  // head vectors per control wave
  static_assert(kTile * 8 == kC && kC % HD == 0, "tile shape");
  static_assert(kMaxChunks <= WAVE, "one lane per chunk in the combine");
  if (!it.valid) return;
  constexpr bool cw = CTRL;
  const int ct = threadIdx.x - kS, wave = ct / WAVE, lane = threadIdx.x % WAVE;
  float* qs = la + A::qs;
  float* kn = la + A::kn;
  float* vn = la + A::vn;
  float* sc = la + A::sc;
  float* st = la + A::st;
  float* wts = la + A::wts;
  float* tiles = la + A::tiles;
  const int G = U(lp->qh) / U(lp->kvh);
  const int g = it.g, s0 = it.s0, s1 = it.s1, nch = it.nch;
  const bool has_new = s1 == P + 1;
  const float* kb = ly.kcache + (size_t)g * U(lp->ctx) * HD;
  const float* vb = ly.vcache + (size_t)g * U(lp->ctx) * HD;

  if constexpr (cw) {
    // q (G heads) and the new key from the QKV output (agent-coherent),
    // norm weights, rotation of position P, and the new value row.
    const float* qkv = U(lp->qkv);
    const float* cs = U(lp->rope) + (size_t)P * HD;
    const int pb = U(lp->pb), po = U(lp->po), pst = U(lp->pst);
    const int nvec = G + (has_new ? 1 : 0);
    const int hp = lane * pst, hq = hp < pb ? hp : 0;
    float xv[MAXV][PER], wv[MAXV][PER], fr[MAXV], fi[MAXV];
#pragma unroll
    for (int j = 0; j < MAXV; j++) {
      const int v = wave + j * kCW;
      const bool key = v == G;
      const float* src = key ? qkv + U(lp->qd) + g * HD : qkv + (size_t)(g * G + (v < G ? v : 0)) * HD;
      const uint16_t* nw = key ? ly.k_norm : ly.q_norm;
      const uint16_t* nws = nw ? nw : (const uint16_t*)U(lp->emb);
#pragma unroll
      for (int i = 0; i < PER; i++) {
        const int e = min(lane + i * WAVE, HD - 1);
        xv[j][i] = cload(src + e);
        wv[j][i] = bf16_to_f32(gload(nws + e));
      }
      fr[j] = gload(cs + hq);
      fi[j] = gload(cs + hq + po);
    }
    const float vnew = cload(qkv + U(lp->qd) + U(lp->kvd) + g * HD + (ct < HD ? ct : 0));
#pragma unroll
    for (int j = 0; j < MAXV; j++) {
      const int v = wave + j * kCW;
      if (v < nvec)
        norm_rope_regs<HD>(xv[j], wv[j], (v == G ? ly.k_norm : ly.q_norm) != nullptr, U(lp->eps), fr[j],
                           fi[j], pb, po, pst, v == G ? kn : qs + v * HD);
    }
    if (has_new && ct < HD) vn[ct] = vnew;
    if (ct < kMaxG) {
      st[ct] = -INFINITY;
      st[kMaxG + ct] = 0.0f;
    }
  }
  const float scale = sqrtf((float)HD);
  // Scores: 8 lanes per key (KP dims each). P.V: thread = output (head h_r,
  // dim d) for r < OPT, summing the tile's keys in order.
  const int kk = ct / 8, pp = ct % 8, d = ct % HD;
  float acc[OPT];
#pragma unroll
  for (int r = 0; r < OPT; r++) acc[r] = 0.0f;

  for (int t0 = s0, buf = 0; t0 < s1; t0 += kTile, buf ^= 1) {
    const int n = min(kTile, s1 - t0);
    float* kt = tiles + buf * 2 * kTile * HD;
    float* vt = kt + kTile * HD;
    csync<true>(cs);  // this tile (and the stage loads) landed; previous tile consumed
    if (cw && t0 + kTile < s1) {
      float* nk = tiles + (buf ^ 1) * 2 * kTile * HD;
      dma_kv<HD>(kb, vb, t0 + kTile, min(kTile, s1 - t0 - kTile), nk, nk + kTile * HD);
    }
    if (has_new && P >= t0 && P < t0 + n) {  // row P: this step's key and value
      if (cw && ct < HD) {
        kt[(P - t0) * HD + ct] = kn[ct];
        vt[(P - t0) * HD + ct] = vn[ct];
      }
      csync<false>(cs);
    }
    if constexpr (cw) {
      float kv[KP];
      lds_vec<KP>(kt + kk * HD + pp * KP, kv);
#pragma unroll 1
      for (int h = 0; h < G; h++) {
        float q[KP];
        lds_vec<KP>(qs + h * HD + pp * KP, q);
        float a = 0.0f;
#pragma unroll
        for (int i = 0; i < KP; i++) a = fmaf(q[i], kv[i], a);
        a = group_sum<8>(a);
        if (pp == 0) sc[h * kTile + kk] = a / scale;
      }
    }
    csync<false>(cs);
    if constexpr (cw) {
      for (int h = wave; h < G; h += kCW) {  // online softmax of head h
        const float s = lane < n ? sc[h * kTile + lane] : -INFINITY;
        const float mo = st[h], mn = fmaxf(mo, wave_max(s));
        const float e = lane < n ? expf(s - mn) : 0.0f;
        if (lane < kTile) sc[h * kTile + lane] = e;  // 0 past the tile's keys
        const float sum = wave_sum(e);
        if (lane == 0) {
          const float f = expf(mo - mn);
          st[2 * kMaxG + h] = f;
          st[kMaxG + h] = st[kMaxG + h] * f + sum;
          st[h] = mn;
        }
      }
    }
    csync<false>(cs);
    if constexpr (cw) {
#pragma unroll
      for (int r = 0; r < OPT; r++) {
        const int h = min((ct + r * kC) / HD, G - 1);
        acc[r] *= st[2 * kMaxG + h];
      }
      for (int key = 0; key < n; key++) {
        const float v = vt[key * HD + d];
#pragma unroll
        for (int r = 0; r < OPT; r++) {
          const int h = min((ct + r * kC) / HD, G - 1);
          acc[r] = fmaf(sc[h * kTile + key], v, acc[r]);
        }
      }
    }
  }
  mark(3);
  if constexpr (cw) {
    float* part = U(lp->part);
    const int mc = U(lp->max_chunks);
#pragma unroll
    for (int r = 0; r < OPT; r++) {
      const int o = ct + r * kC, h = o / HD;
      if (o < G * HD) {
        float* pp2 = part + ((size_t)(g * G + h) * mc + it.c) * (HD + 2);
        cstore(pp2 + 2 + d, acc[r]);
        if (d == 0) {
          cstore(pp2, st[h]);
          cstore(pp2 + 1, st[kMaxG + h]);
        }
      }
    }
    if (has_new && ct < HD) {  // cache row P of kv head g, read by later steps
      gstore(ly.kcache + ((size_t)g * U(lp->ctx) + P) * HD + ct, kn[ct]);
      gstore(ly.vcache + ((size_t)g * U(lp->ctx) + P) * HD + ct, vn[ct]);
    }
  }
  csync<true>(cs);  // partials stored
  if (threadIdx.x == kS) {
    const unsigned done =
        __hip_atomic_fetch_add((__attribute__((address_space(1))) unsigned*)(U(lp->att_cnt) + g), 1u,
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    flag[0] = done == (unsigned)(nch - 1);
  }
  csync<false>(cs);
  if (!U(flag[0])) {
    mark(4);
    return;
  }

  // Last worker of kv head g: combine its G heads, one output per control
  // thread per round.
  const float* part = U(lp->part);
  const int mc = U(lp->max_chunks);
  float m[MAXV], l[MAXV];
#pragma unroll
  for (int j = 0; j < MAXV; j++) {
    const int h = wave + j * kCW;
    const float* pb = part + ((size_t)(g * G + (h < G ? h : 0)) * mc + (lane < nch ? lane : 0)) * (HD + 2);
    m[j] = cw ? cload(pb) : 0.0f;
    l[j] = cw ? cload(pb + 1) : 0.0f;
  }
  for (int o0 = 0; o0 < G * HD; o0 += kC) {
    float x[1][kMaxChunks];
    if constexpr (cw) {
#pragma unroll
      for (int r = 0; r < 1; r++) {
        const int o = min(o0 + ct + r * kC, G * HD - 1), h = o / HD, dd = o % HD;
        const float* pb = part + (size_t)(g * G + h) * mc * (HD + 2) + 2 + dd;
#pragma unroll
        for (int i = 0; i < kMaxChunks; i++) x[r][i] = cload(pb + (size_t)(i < nch ? i : 0) * (HD + 2));
      }
    }
    if (o0 == 0) {
      if constexpr (cw) {
#pragma unroll
        for (int j = 0; j < MAXV; j++) {
          const int h = wave + j * kCW;
          if (h < G) {
            const float mj = lane < nch ? m[j] : -INFINITY;
            const float M = wave_max(mj);
            const float w = lane < nch ? expf(mj - M) : 0.0f;
            if (lane < kMaxChunks) wts[h * (kMaxChunks + 1) + lane] = w;
            const float wl = wave_sum(lane < nch ? w * l[j] : 0.0f);
            if (lane == 0) wts[h * (kMaxChunks + 1) + kMaxChunks] = wl;
          }
        }
      }
      csync<false>(cs);
    }
    if constexpr (cw) {
#pragma unroll
      for (int r = 0; r < 1; r++) {
        const int o = o0 + ct + r * kC, h = o / HD, dd = o % HD;
        if (o < G * HD) {
          const float* w = wts + h * (kMaxChunks + 1);
          float a = 0.0f;
#pragma unroll
          for (int i = 0; i < kMaxChunks; i++)
            if (i < nch) a = fmaf(w[i], x[r][i], a);
          cstore(U(lp->att) + (size_t)(g * G + h) * HD + dd, a / w[kMaxChunks]);
        }
      }
    }
  }
  if (threadIdx.x == kS)
    __hip_atomic_store((__attribute__((address_space(1))) unsigned*)(U(lp->att_cnt) + g), 0u,
                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  mark(4);
}

// -------------------------------------------------------------- argmax --

__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
  // Larger value wins; equal values keep the lower index. NaN never wins.
  return v > bv || (v == bv && i < bi);
}

__device__ __forceinline__ void wave_best(float& bv, int& bi) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(bv, off, WAVE);
    const int oi = __shfl_xor(bi, off, WAVE);
    if (better(ov, oi, bv, bi)) {
      bv = ov;
      bi = oi;
    }
  }
}

// ---------------------------------------------------------------- step --

// Phase tracer, on the first worker (block 1) when enabled, kept by the
// first control thread: time before each barrier (work, row 0), inside it
// (wait, row 1), and for the phase after it the end of input staging
// (row 2), weight loop (3) and epilogue (4); for attention, the end of the
// key tiles (3) and of the item (4). Accumulated in LDS (no global memory
// traffic of its own between barriers) and added to the global trace at the
// end of the launch.
struct Tracer {
  unsigned long long* acc;  // LDS, block 1 only; null: off
  int k, nbar;
  uint64_t last;
};

__device__ __forceinline__ void mark(const Tracer& tr, int which) {
  if (tr.acc && threadIdx.x == kS && tr.k > 0)
    tr.acc[which * tr.nbar + tr.k - 1] += wall_clock64() - tr.last;
}

// Stream-wave marks (rows 5-7), by thread 0, against the phase start that
// the first control thread publishes in LDS (`t0`) at each barrier.
__device__ __forceinline__ void mark_stream(const Tracer& tr, const unsigned long long* t0, int which) {
  if (tr.acc && threadIdx.x == 0 && tr.k > 0)
    tr.acc[which * tr.nbar + tr.k - 1] += wall_clock64() - *(volatile const unsigned long long*)t0;
}

// Control-wave side of a phase boundary: arrive, issue the next phase's
// control loads (`prefetch`), wait.
template <typename F>
__device__ __forceinline__ void phase_boundary(GridSync& g, CSync& cs, Tracer& tr, unsigned long long* tpub,
                                               F prefetch) {
  const bool on = tr.acc && threadIdx.x == kS;
  uint64_t t0 = 0;
  if (on) t0 = wall_clock64();
  worker_arrive(g, cs);
  prefetch();
  worker_wait(g, cs);  // every control wave, outside any divergent branch
  if (on) {
    const uint64_t t1 = wall_clock64();
    tr.acc[tr.k] += t0 - tr.last;
    tr.acc[tr.nbar + tr.k] += t1 - t0;
    tr.last = t1;
    // phase start for the stream waves' marks (read after the next block barrier)
    *(volatile unsigned long long*)tpub = t1;
  }
  tr.k++;
}

// Layer descriptor l, from the table copied into LDS at kernel start (a
// global read here would cost a memory round trip at every phase).
__device__ __forceinline__ DecodeLayer layer_at(const DecodeParams* lp, int l) {
  const DecodeLayer* tab =
      (const DecodeLayer*)((const float*)lp + kParamFloats + U(lp->layer_lds));
  const DecodeLayer& t = tab[l];
  DecodeLayer ly;
  ly.qkv = U(t.qkv);
  ly.o = U(t.o);
  ly.gate = U(t.gate);
  ly.up = U(t.up);
  ly.down = U(t.down);
  ly.attn_norm = U(t.attn_norm);
  ly.ffn_norm = U(t.ffn_norm);
  ly.q_norm = U(t.q_norm);
  ly.k_norm = U(t.k_norm);
  ly.kcache = U(t.kcache);
  ly.vcache = U(t.vcache);
  return ly;
}

// Phases of a step: kDecodePhases per layer (QKV, attention, O, gate/up,
// down), then the logits.
enum PhaseKind { PH_QKV, PH_ATTN, PH_O, PH_GU, PH_DOWN, PH_LOGITS };
static_assert(PH_LOGITS == kDecodePhases, "phases per layer");

__device__ __forceinline__ int phase_kind(int ph, int L) {
  return ph == kDecodePhases * L ? PH_LOGITS : ph % kDecodePhases;
}

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
  const int l = ph / kDecodePhases;
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

// Next GEMV phase after ph (attention phases skipped), or -1 after the
// logits.
__device__ __forceinline__ int next_gemv(int ph, int L) {
  if (ph >= kDecodePhases * L) return -1;
  const int nx = ph + 1;
  return phase_kind(nx, L) == PH_ATTN ? nx + 1 : nx;
}

// Epilogue of a GEMV phase, by the control waves: row results (slice sums
// added in slice order) to the phase's output.
__device__ __forceinline__ void gemv_epilogue(const DecodeParams* lp, const GemvPhase& gp, int w,
                                              int NW, const float* part1, const float* part2,
                                              const float* xown, float* red, CSync& cs) {
  constexpr bool cw = true;
  const int ct = threadIdx.x - kS;
  const int S = gp.plan.S, row0 = w * gp.plan.rb;
  const int rows = max(0, min(gp.plan.rb, gp.N - row0));
  float bv = -INFINITY;
  int bi = U(lp->V);
  if constexpr (cw) {
    for (int r = ct; r < rows; r += kC) {
      float y = 0.0f, y2 = 0.0f;
      for (int s = 0; s < S; s++) {
        y += part1[r * S + s];
        if (gp.w2) y2 += part2[r * S + s];
      }
      const int row = row0 + r;
      switch (gp.epi) {
        case EPI_QKV: cstore(U(lp->qkv) + row, y); break;
        case EPI_RESIDUAL: cstore(U(lp->x) + row, xown[r] + y); break;
        case EPI_SWIGLU: cstore(U(lp->act) + row, silu_mul(y, y2)); break;
        default:  // EPI_LOGITS
          if (U(lp->logits)) gstore(U(lp->logits) + row, y);
          if (row == 0) cstore(U(lp->am_v) + NW, y);  // logits[0] for the NaN rule
          if (better(y, row, bv, bi)) {
            bv = y;
            bi = row;
          }
      }
    }
  }
  if (gp.epi == EPI_LOGITS) {
    if constexpr (cw) {
      wave_best(bv, bi);
      if (threadIdx.x % WAVE == 0) {
        red[ct / WAVE] = bv;
        ((int*)red)[kCW + ct / WAVE] = bi;
      }
    }
    csync<false>(cs);
    if (threadIdx.x == kS) {
      for (int i = 1; i < kCW; i++) {
        const float v = red[i];
        const int j = ((int*)red)[kCW + i];
        if (better(v, j, bv, bi)) {
          bv = v;
          bi = j;
        }
      }
      cstore(U(lp->am_v) + w, bv);
      cstore(U(lp->am_i) + w, bi);
    }
  }
}

// LDS of a worker block (after the parameter copy).
struct WorkerLds {
  float* red;                // [64]: reductions
  int* flag;                 // attention: last-worker flag
  unsigned* cbar;            // control-wave barrier counter
  unsigned long long* tpub;  // phase start, for the tracer
  float* xown;               // [kOwnMax] residual rows
  float* un;                 // region shared by the GEMV and attention phases
  float *part1, *part2, *xs; // GEMV: slice sums first (constant LDS addresses), input row
};

__device__ __forceinline__ WorkerLds worker_lds(float* lds) {
  WorkerLds m;
  m.red = lds;
  m.flag = (int*)(lds + 64);
  m.cbar = (unsigned*)(lds + 65);
  m.tpub = (unsigned long long*)(lds + 66);
  m.xown = lds + kCtl;
  m.un = m.xown + kOwnMax;
  m.part1 = m.un;
  m.part2 = m.part1 + kDecodePartMax;
  m.xs = m.part2 + kDecodePartMax;
  return m;
}

// Stream waves: the GEMV phases only. Two block barriers per GEMV phase are
// shared with the control waves: "input row staged" (end of stage_input)
// and "slice sums written". Right after the second the next GEMV phase's
// first two batches are issued (this may stall while the memory queues are
// full, which holds back no other wave).
__device__ __forceinline__ void stream_loop(const DecodeParams* lp, const WorkerLds& m, Tracer& tr, int tok,
                                            int w) {
  const int L = U(lp->L);
  Batch b0, b1;
  Cursor ld{0, 0, 0};
  Job job;
  {
    const GemvPhase gp = gemv_phase(lp, 0, tok);
    job = make_job(gp.w, gp.w2, gp.N, gp.K, gp.plan, w);
    gemv_prefetch_any(job, ld, b0, b1);
  }
  for (int ph = 0; ph >= 0; ph = next_gemv(ph, L)) {
    bar<false>();  // input row staged
    mark_stream(tr, m.tpub, 5);
    if (job.w2)
      gemv_run<true>(job, b0, b1, ld, m.xs, m.part1, m.part2);
    else
      gemv_run<false>(job, b0, b1, ld, m.xs, m.part1, m.part2);
    mark_stream(tr, m.tpub, 6);
    bar<false>();  // slice sums written
    const int nx = next_gemv(ph, L);
    ld = Cursor{0, 0, 0};
    if (nx >= 0) {
      const GemvPhase np = gemv_phase(lp, nx, tok);
      job = make_job(np.w, np.w2, np.N, np.K, np.plan, w);
      gemv_prefetch_any(job, ld, b0, b1);
    }
    mark_stream(tr, m.tpub, 7);
    // the tracer's phase count follows the control waves' barriers
    tr.k += nx >= 0 && phase_kind(ph + 1, L) == PH_ATTN ? 2 : 1;
  }
}

// Control waves: every phase (staging, epilogues, attention, grid
// barriers), synchronising among themselves with csync and with the stream
// waves only at the two block barriers of each GEMV phase.
template <int HD>
__device__ __forceinline__ void control_loop(const DecodeParams* lp, const WorkerLds& m, GridSync& g,
                                             Tracer& tr, int P, int tok, int w, int NW) {
  const int L = U(lp->L);
  CSync cs{m.cbar, 0u, g.err};
  auto mk = [&](int which) { mark(tr, which); };
  const int last = kDecodePhases * L;  // the logits phase
  for (int ph = 0;; ph++) {
    const int kind = phase_kind(ph, L);
    if (kind == PH_ATTN) {
      attention_phase<HD>(lp, layer_at(lp, ph / kDecodePhases), P, attn_item(lp, P, w), m.un, m.flag, cs, mk);
    } else {
      const GemvPhase gp = gemv_phase(lp, ph, tok);
      // Residual rows kept from this input: those the next residual phase
      // (O after QKV, down after gate/up) updates.
      int own0 = 0, nown = 0;
      if (kind == PH_QKV || kind == PH_GU) {
        const DecodeGemvPlan pr = kind == PH_QKV ? U(lp->p_o) : U(lp->p_down);
        own0 = w * pr.rb;
        nown = max(0, min(pr.rb, U(lp->d) - own0));
      }
      // hidden-state capture: x entering layer l (l > 0) is layer l-1's
      // output; x entering the logits is the last layer's
      float *cap_raw = nullptr, *cap_norm = nullptr;
      if (U(lp->cap) && w == 0 && (kind == PH_QKV || kind == PH_LOGITS) && ph > 0) {
        cap_raw = U(lp->cap) + (size_t)(ph / kDecodePhases - 1) * U(lp->d);
        if (kind == PH_LOGITS) cap_norm = U(lp->cap_final);
      }
      stage_input(gp.src, gp.emb, gp.K, gp.nw, U(lp->eps), m.xs, m.red, m.xown, own0, nown, cap_raw,
                  cap_norm, cs);
      mk(2);
      bar<false>();  // slice sums written
      mk(3);
      gemv_epilogue(lp, gp, w, NW, m.part1, m.part2, m.xown, m.red, cs);
      mk(4);
    }
    if (ph == last) break;
    const int nx = ph + 1;
    phase_boundary(g, cs, tr, m.tpub, [&] {
      if (phase_kind(nx, L) == PH_ATTN) {
        // the item's first K/V tile (rows of earlier steps) goes to LDS
        const AttnItem item = attn_item(lp, P, w);
        if (item.valid) {
          using A = AttLds<HD>;
          const DecodeLayer ly = layer_at(lp, nx / kDecodePhases);
          float* kt = m.un + A::tiles;
          dma_kv<HD>(ly.kcache + (size_t)item.g * U(lp->ctx) * HD,
                     ly.vcache + (size_t)item.g * U(lp->ctx) * HD, item.s0,
                     min(kTile, item.s1 - item.s0), kt, kt + kTile * HD);
        }
      }
    });
  }
  phase_boundary(g, cs, tr, m.tpub, [] {});
}

// The parameters are read from device memory (not kernel arguments) and
// copied to LDS: the compiler reloads them per use instead of keeping
// dozens of them live in scalar registers for the whole step.
template <int HD>
__global__ __launch_bounds__(kT, 1) void decode_step_kernel(const DecodeParams* params) {
  extern __shared__ __attribute__((aligned(16))) float lds_all[];
  {
    const unsigned* src = (const unsigned*)params;
    for (int i = threadIdx.x; i < (int)(sizeof(DecodeParams) / 4); i += kT)
      ((unsigned*)lds_all)[i] = src[i];
    __syncthreads();
    // the layer table, after the block's working LDS
    const DecodeParams* lp0 = (const DecodeParams*)lds_all;
    const DecodeLayer* tab = U(lp0->layers);
    DecodeLayer* dst = (DecodeLayer*)(lds_all + kParamFloats + U(lp0->layer_lds));
    for (int i = threadIdx.x; i < U(lp0->L); i += kT) dst[i] = tab[i];
    __syncthreads();
  }
  const DecodeParams* lp = (const DecodeParams*)lds_all;
  float* lds = lds_all + kParamFloats;
  // master's reduction slots
  float* part1 = lds + kCtl + kOwnMax;
  float* part2 = part1 + kDecodePartMax;

  GridSync g{U(lp->sync_state), U(lp->sync_err), (unsigned)cload((const int*)U(lp->epoch)) + 1u};
  const int P = cload(U(lp->pos)), tok = cload(U(lp->tok));
  const int L = U(lp->L);
  const int nbar = decode_barriers(L);

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
    wave_best(bv, bi);
    if (threadIdx.x % WAVE == 0) {
      part1[threadIdx.x / WAVE] = bv;
      ((int*)part2)[threadIdx.x / WAVE] = bi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
      for (int i = 1; i < kT / WAVE; i++)
        if (better(part1[i], ((int*)part2)[i], bv, bi)) {
          bv = part1[i];
          bi = ((int*)part2)[i];
        }
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
  const WorkerLds m = worker_lds(lds);
  if (threadIdx.x == 0) *m.cbar = 0u;
  __syncthreads();
  if (control_wave())
    control_loop<HD>(lp, m, g, tr, P, tok, w, NW);
  else
    stream_loop(lp, m, tr, tok, w);
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

size_t att_lds_floats(int hd) {
  switch (hd) {
    case 16: return AttLds<16>::total;
    case 32: return AttLds<32>::total;
    case 64: return AttLds<64>::total;
    case 128: return AttLds<128>::total;
    default: return 0;
  }
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

// LDS floats of the block's working area (after the parameter copy); the
// layer table follows it.
size_t decode_work_floats(const DecodeParams& p) {
  const size_t kmax = std::max(p.d, std::max(p.qd, p.H));
  const size_t gemv = kmax + 2 * kDecodePartMax;
  const size_t att = att_lds_floats(p.hd);
  return kCtl + kOwnMax + std::max(gemv, att);
}

size_t decode_lds_bytes(const DecodeParams& p) {
  const size_t floats = decode_work_floats(p) + (size_t)p.L * (sizeof(DecodeLayer) / sizeof(float));
  return std::max(kMinLds, floats * sizeof(float));
}

bool decode_supported(int L, int d, int H, int qh, int kvh, int hd, int qd, int V, int blocks,
                      size_t lds_limit) {
  if (hd != 16 && hd != 32 && hd != 64 && hd != 128) return false;
  const int workers = blocks - 1;
  if (L < 1 || workers < 1 || kvh <= 0 || qh % kvh || qh / kvh > kMaxG || kvh > workers) return false;
  if (d % 8 || H % 8 || qd % 8 || d < 8) return false;
  if ((V + workers - 1) / workers > kDecodePartMax) return false;
  if ((d + workers - 1) / workers > kOwnMax) return false;
  DecodeParams p{};
  p.L = L;
  p.d = d;
  p.H = H;
  p.qd = qd;
  p.hd = hd;
  return kParamFloats * sizeof(float) + decode_lds_bytes(p) <= lds_limit;
}

int decode_max_chunks(int kvh, int blocks) {
  return std::max(1, std::min(kMaxChunks, (blocks - 1) / std::max(1, kvh)));
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
  if (p.max_chunks <= 0 || p.max_chunks > kMaxChunks || p.max_chunks * p.kvh > blocks - 1)
    ST_DIE("decode step: bad attention chunking");
  if (!p.att_cnt) ST_DIE("decode step: attention counters missing");
  if (p.pst < 1 || (p.pb + p.pst - 1) / p.pst > WAVE || p.pb - p.pst + p.po >= p.hd)
    ST_DIE("decode step: RoPE pairs must fit one per lane within the head");
  if (p.p_o.rb > kOwnMax || p.p_down.rb > kOwnMax) ST_DIE("decode step: too many residual rows per block");
  if (p.layer_lds != (int)decode_work_floats(p)) ST_DIE("decode step: layer table offset mismatch");
  switch (p.hd) {
    case 16: launch<16>(p, dp, blocks, s); break;
    case 32: launch<32>(p, dp, blocks, s); break;
    case 64: launch<64>(p, dp, blocks, s); break;
    case 128: launch<128>(p, dp, blocks, s); break;
    default: ST_DIE("decode step supports head_dim 16, 32, 64 or 128");
  }
}

}  // namespace sg
