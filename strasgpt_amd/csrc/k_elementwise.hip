// Small fused kernels of the forward pass: embedding gather, row RMSNorm,
// per-head QK RMSNorm + RoPE, and the greedy argmax over the vocabulary.
#include "device_common.h"
#include "hip_check.h"
#include "kernels.h"

namespace sg {

namespace {

// Reference source/transformer.c:1247-1255: x[t][e] = bf16 -> f32 of the
// token's embedding row (exact). One 16-byte load (8 values) per thread,
// grid (T, d / 2048 rounded up): one memory latency per row (a block-strided
// loop over the row waited one per 256 values: 10.9 against 2.9 us for a
// decode step's row at d = 5120).
__global__ __launch_bounds__(256) void embed8_kernel(const int* tok, const uint16_t* table, int d, float* x) {
  const int t = blockIdx.x, e = (blockIdx.y * 256 + threadIdx.x) * 8;
  if (e >= d) return;
  const uint4 w = *(const uint4*)(table + (size_t)tok[t] * d + e);
  float* xr = x + (size_t)t * d + e;
  *(float4*)xr = make_float4(bf16_lo(w.x), bf16_hi(w.x), bf16_lo(w.y), bf16_hi(w.y));
  *(float4*)(xr + 4) = make_float4(bf16_lo(w.z), bf16_hi(w.z), bf16_lo(w.w), bf16_hi(w.w));
}

// Reference rmsnorm (source/transformer.c:978-999) on one row per block.
__global__ __launch_bounds__(256) void rmsnorm_kernel(const float* x, const uint16_t* w,
                                                      float* y, int d, float eps) {
  __shared__ float red[4];
  const float* xr = x + (size_t)blockIdx.x * d;
  float* yr = y + (size_t)blockIdx.x * d;
  float ss = 0.0f;
  for (int e = threadIdx.x; e < d; e += 256) ss = fmaf(xr[e], xr[e], ss);
  const float s = rms_scale(block_sum<256>(ss, red), d, eps);
  for (int e = threadIdx.x; e < d; e += 256) yr[e] = (xr[e] * s) * bf16_to_f32(w[e]);
}

// Residual add of a split-K projection and RMSNorm of the updated row. The
// split partial sums are added in split order first, so x gains one
// rounded term like the reference's x += dot (source/transformer.c:
// 1439-1445, 1498-1504); an MoE layer's routed sum (the weighted expert
// outputs, fmaf-chained in top-k order) is added the same way; then the
// reference RMSNorm (source/transformer.c:
// 978-999) is written as fp32 and/or as the bf16 hi/lo planes that the next
// GEMM consumes (hi = bf16(y), lo = bf16(y - hi)).
// One block per row, the row held in registers (NV float4 per thread,
// d <= 1024 NV): x and every split's partial are loaded before any is
// used, then one reduction and the normalised stores. Partials are added in
// split order.
template <int NV>
__global__ __launch_bounds__(256) void residual_norm_kernel(NormParams p) {
  __shared__ float red[4];
  const int row = blockIdx.x, d4 = p.d / 4, tid = threadIdx.x;
  float4* xr = (float4*)(p.x + (size_t)row * p.d);
  float4 v[NV];
#pragma unroll
  for (int i = 0; i < NV; i++) {
    const int e = tid + 256 * i;
    v[i] = e < d4 ? xr[e] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  if (p.splits > 0) {
    float4 o[NV];
    const float4* p0 = (const float4*)(p.part + (size_t)row * p.d);
#pragma unroll
    for (int i = 0; i < NV; i++) {
      const int e = tid + 256 * i;
      o[i] = e < d4 ? p0[e] : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    // UB splits' loads in flight before their sums, added in split order
    // (one at a time for rows of more than 3072: four would cost waves per
    // SIMD, measured 44 -> 47 us on 2048 rows of 5120 with 3 splits)
    constexpr int UB = NV <= 3 ? 4 : 1;
    for (int sp = 1; sp < p.splits; sp += UB) {
      float4 q[UB][NV];
#pragma unroll
      for (int u = 0; u < UB; u++) {
        const float4* ps = (const float4*)(p.part + ((size_t)min(sp + u, p.splits - 1) * p.rows + row) * p.d);
#pragma unroll
        for (int i = 0; i < NV; i++) q[u][i] = ps[min(tid + 256 * i, d4 - 1)];
      }
#pragma unroll
      for (int u = 0; u < UB; u++) {
        if (sp + u >= p.splits) break;
#pragma unroll
        for (int i = 0; i < NV; i++) {
          if (tid + 256 * i < d4) {
            o[i].x += q[u][i].x;
            o[i].y += q[u][i].y;
            o[i].z += q[u][i].z;
            o[i].w += q[u][i].w;
          }
        }
      }
    }
#pragma unroll
    for (int i = 0; i < NV; i++) {
      const int e = tid + 256 * i;
      if (e < d4) {
        v[i].x += o[i].x;
        v[i].y += o[i].y;
        v[i].z += o[i].z;
        v[i].w += o[i].w;
        xr[e] = v[i];
      }
    }
  }
  if (p.routed) {
    float4 acc[NV];
#pragma unroll
    for (int i = 0; i < NV; i++) acc[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    // UB experts' rows in flight before their products, in top-k order
    constexpr int UB = NV <= 3 ? 4 : 1;
    for (int j = 0; j < p.topk; j += UB) {
      float4 q[UB][NV];
      float wj[UB];
#pragma unroll
      for (int u = 0; u < UB; u++) {
        const size_t slot = (size_t)row * p.topk + min(j + u, p.topk - 1);
        wj[u] = p.routed_w[slot];
        const float4* oj = (const float4*)(p.routed + slot * p.d);
#pragma unroll
        for (int i = 0; i < NV; i++) q[u][i] = oj[min(tid + 256 * i, d4 - 1)];
      }
#pragma unroll
      for (int u = 0; u < UB; u++) {
        if (j + u >= p.topk) break;
#pragma unroll
        for (int i = 0; i < NV; i++) {
          if (tid + 256 * i < d4) {
            acc[i].x = fmaf(wj[u], q[u][i].x, acc[i].x);
            acc[i].y = fmaf(wj[u], q[u][i].y, acc[i].y);
            acc[i].z = fmaf(wj[u], q[u][i].z, acc[i].z);
            acc[i].w = fmaf(wj[u], q[u][i].w, acc[i].w);
          }
        }
      }
    }
#pragma unroll
    for (int i = 0; i < NV; i++) {
      const int e = tid + 256 * i;
      if (e < d4) {
        v[i].x += acc[i].x;
        v[i].y += acc[i].y;
        v[i].z += acc[i].z;
        v[i].w += acc[i].w;
        xr[e] = v[i];
      }
    }
  }
  if (!p.w) return;
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; i++) {
    ss = fmaf(v[i].x, v[i].x, ss);
    ss = fmaf(v[i].y, v[i].y, ss);
    ss = fmaf(v[i].z, v[i].z, ss);
    ss = fmaf(v[i].w, v[i].w, ss);
  }
  const float s = rms_scale(block_sum<256>(ss, red), p.d, p.eps);
#pragma unroll
  for (int i = 0; i < NV; i++) {
    const int e = tid + 256 * i;
    if (e >= d4) continue;
    const uint2 w2 = *(const uint2*)(p.w + 4 * e);
    const float wv[4] = {__uint_as_float(w2.x << 16), __uint_as_float(w2.x & 0xFFFF0000u),
                         __uint_as_float(w2.y << 16), __uint_as_float(w2.y & 0xFFFF0000u)};
    const float xv[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
    float y[4];
#pragma unroll
    for (int j = 0; j < 4; j++) y[j] = (xv[j] * s) * wv[j];
    const size_t idx = (size_t)row * p.d + 4 * e;
    if (p.y) *(float4*)(p.y + idx) = make_float4(y[0], y[1], y[2], y[3]);
    if (p.y_hi) {
      uint16_t h[4], l[4];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        h[j] = f32_to_bf16_rne(y[j]);
        l[j] = f32_to_bf16_rne(y[j] - bf16_to_f32(h[j]));
      }
      *(uint2*)(p.y_hi + idx) = make_uint2(h[0] | ((unsigned)h[1] << 16), h[2] | ((unsigned)h[3] << 16));
      if (p.y_lo) *(uint2*)(p.y_lo + idx) = make_uint2(l[0] | ((unsigned)l[1] << 16), l[2] | ((unsigned)l[3] << 16));
    }
  }
}

// One wavefront per (token, head): optional per-head RMSNorm with the
// layer's q/k norm weight (source/transformer.c:1293-1307, 1340-1356), then
// the pair rotation v0' = v0 cos - v1 sin, v1' = v0 sin + v1 cos with the
// host-built table (source/transformer.c:1309-1323, 1358-1373). With a bf16
// cache (kstage given) a key row is read from kstage and the whole result
// row is stored rounded into the cache.
__global__ __launch_bounds__(64) void qk_norm_rope_kernel(
    float* q, int q_heads, float* kcache, int ctx, int hd, const int* pos,
    const uint16_t* qn, const uint16_t* kn, float eps, const float* rope,
    int pair_bound, int pair_offset, int pair_stride, const float* kstage) {
#pragma clang fp contract(off)
  __shared__ float v[512];
  const int t = blockIdx.x, head = blockIdx.y, lane = threadIdx.x;
  const int P = *pos + t;
  const bool staged = kstage && head >= q_heads;
  float* row;
  const float* src;
  const uint16_t* nw;
  if (head < q_heads) {
    row = q + ((size_t)t * q_heads + head) * hd;
    src = row;
    nw = qn;
  } else {
    const int kh = head - q_heads;
    row = kcache + ((size_t)kh * ctx + P) * hd;  // a bf16 row when staged
    src = staged ? kstage + ((size_t)t * (gridDim.y - q_heads) + kh) * hd : row;
    nw = kn;
  }
  float ss = 0.0f;
  for (int e = lane; e < hd; e += WAVE) {
    const float x = src[e];
    v[e] = x;
    ss = fmaf(x, x, ss);
  }
  ss = wave_sum(ss);
  if (nw) {
    const float s = rms_scale(ss, hd, eps);
    for (int e = lane; e < hd; e += WAVE) v[e] = (v[e] * s) * bf16_to_f32(nw[e]);
  }
  __syncthreads();
  const float* cs = rope + (size_t)P * hd;
  if (!staged) {
    for (int i = lane; i * pair_stride < pair_bound; i += WAVE) {
      const int h = i * pair_stride;
      const float fr = cs[h], fi = cs[h + pair_offset];
      const float v0 = v[h], v1 = v[h + pair_offset];
      row[h] = v0 * fr - v1 * fi;
      row[h + pair_offset] = v0 * fi + v1 * fr;
    }
    return;
  }
  // staged key: rotate in LDS (each pair read and written by one lane), then
  // store every element rounded
  for (int i = lane; i * pair_stride < pair_bound; i += WAVE) {
    const int h = i * pair_stride;
    const float fr = cs[h], fi = cs[h + pair_offset];
    const float v0 = v[h], v1 = v[h + pair_offset];
    v[h] = v0 * fr - v1 * fi;
    v[h + pair_offset] = v0 * fi + v1 * fr;
  }
  __syncthreads();
  uint16_t* row16 = (uint16_t*)kcache + ((size_t)(head - q_heads) * ctx + P) * hd;
  for (int e = lane; e < hd; e += WAVE) row16[e] = f32_to_bf16_any(v[e]);
}

// The same for head sizes 16-128 with at most one rotated pair per lane,
// four heads per block (one per wavefront; the loop form's one-wavefront
// blocks are dispatched slower than they finish), with every load of the
// wavefront (the row, the norm weights, the lane's rotation) issued before
// the first is used: the loop form waits a memory latency per step (row,
// then weights, then rotation). Same arithmetic in the same order.
// PLANES: a key head's wavefront also writes its finished key and the
// value row of position P into the attention operand planes (hi/lo bf16
// parts, as split_rows_kernel), for short prompts in place of that launch.
constexpr int kQkrHeads = 4;
template <int HD, bool PLANES>
__global__ __launch_bounds__(kQkrHeads * WAVE) void qk_norm_rope_hd_kernel(
    float* q, int q_heads, int heads, float* kcache, int ctx, const int* pos, const uint16_t* qn,
    const uint16_t* kn, float eps, const float* rope, int pair_bound, int pair_offset, int pair_stride,
    const float* kstage, PlaneRows pl) {
#pragma clang fp contract(off)
  constexpr int PER = (HD + WAVE - 1) / WAVE;
  __shared__ float vsh[kQkrHeads][HD];
  const int lane = threadIdx.x % WAVE, wave = threadIdx.x / WAVE;
  const int t = blockIdx.x, head = blockIdx.y * kQkrHeads + wave;
  if (head >= heads) return;  // (no block-wide barrier below)
  float* v = vsh[wave];
  const int P = *pos + t;
  const bool staged = kstage && head >= q_heads;
  float* row;
  const float* src;
  const uint16_t* nw;
  if (head < q_heads) {
    row = q + ((size_t)t * q_heads + head) * HD;
    src = row;
    nw = qn;
  } else {
    const int kh = head - q_heads;
    row = kcache + ((size_t)kh * ctx + P) * HD;  // a bf16 row when staged
    src = staged ? kstage + ((size_t)t * (heads - q_heads) + kh) * HD : row;
    nw = kn;
  }
  float xv[PER], wv[PER], vv[PER];
#pragma unroll
  for (int i = 0; i < PER; i++) {
    const int e = lane + i * WAVE;
    xv[i] = e < HD ? src[e] : 0.0f;
    wv[i] = nw && e < HD ? bf16_to_f32(nw[e]) : 1.0f;
  }
  const int kh = head - q_heads;
  if (PLANES && head >= q_heads) {  // the value row of position P
    const size_t at = ((size_t)kh * ctx + P) * HD;
#pragma unroll
    for (int i = 0; i < PER; i++) {
      const int e = min(lane + i * WAVE, HD - 1);
      vv[i] = pl.kv_bf16 ? bf16_to_f32(((const uint16_t*)pl.vcache)[at + e]) : ((const float*)pl.vcache)[at + e];
    }
  }
  const int h = lane * pair_stride;
  const bool pair = h < pair_bound;
  const float* cs = rope + (size_t)P * HD;
  const float fr = pair ? cs[h] : 1.0f, fi = pair ? cs[h + pair_offset] : 0.0f;
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < PER; i++)
    if (lane + i * WAVE < HD) ss = fmaf(xv[i], xv[i], ss);
  ss = wave_sum(ss);
  const float s = nw ? rms_scale(ss, HD, eps) : 1.0f;
#pragma unroll
  for (int i = 0; i < PER; i++) {
    const int e = lane + i * WAVE;
    if (e < HD) v[e] = nw ? (xv[i] * s) * wv[i] : xv[i];
  }
  // the wavefront's LDS writes before its reads of other lanes' elements
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  float r0 = 0.0f, r1 = 0.0f;
  if (pair) {
    const float v0 = v[h], v1 = v[h + pair_offset];
    r0 = v0 * fr - v1 * fi;
    r1 = v0 * fi + v1 * fr;
  }
  if (!staged) {
    if (pair) {
      row[h] = r0;
      row[h + pair_offset] = r1;
    }
    if (!PLANES || head < q_heads) return;
  }
  // a staged key (stored rounded) or a key with plane rows: the rotated row
  // in LDS, then every element
  __builtin_amdgcn_wave_barrier();
  if (pair) {
    v[h] = r0;
    v[h + pair_offset] = r1;
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  uint16_t* row16 = (uint16_t*)kcache + ((size_t)(head - q_heads) * ctx + P) * HD;
  const size_t kat = ((size_t)kh * ctx + P) * HD, vat = (size_t)kh * HD * pl.ctx_pad + P;
#pragma unroll
  for (int i = 0; i < PER; i++) {
    const int e = lane + i * WAVE;
    if (e < HD) {
      // the key as the cache holds it (rounded to bf16 when staged), split
      uint32_t hk, lk, hv, lv;
      if (staged) {
        const uint16_t b = f32_to_bf16_any(v[e]);
        row16[e] = b;
        hk = b;
        lk = 0u;
      } else {
        split2(v[e], 0.0f, hk, lk);
      }
      if (PLANES) {
        split2(vv[i], 0.0f, hv, lv);  // (exact hi, zero lo for a bf16 value)
        pl.khi[kat + e] = (uint16_t)hk;
        pl.klo[kat + e] = (uint16_t)lk;
        pl.vthi[vat + (size_t)e * pl.ctx_pad] = (uint16_t)hv;
        pl.vtlo[vat + (size_t)e * pl.ctx_pad] = (uint16_t)lv;
      }
    }
  }
}

// ------------------------------------------------------------- argmax --
constexpr int kArgmaxBlocks = 512;

__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
  // Larger value wins; equal values keep the lower index. NaN never wins.
  return v > bv || (v == bv && i < bi);
}

// Per-block (value, index) of the best element of a contiguous slice.
__device__ void block_best(float& bv, int& bi, float* sv, int* si) {
  sv[threadIdx.x] = bv;
  si[threadIdx.x] = bi;
  __syncthreads();
  for (int st = 128; st > 0; st >>= 1) {
    if (threadIdx.x < st &&
        better(sv[threadIdx.x + st], si[threadIdx.x + st], sv[threadIdx.x], si[threadIdx.x])) {
      sv[threadIdx.x] = sv[threadIdx.x + st];
      si[threadIdx.x] = si[threadIdx.x + st];
    }
    __syncthreads();
  }
  bv = sv[0];
  bi = si[0];
}

__global__ __launch_bounds__(256) void argmax_partial_kernel(ArgmaxParams p) {
  __shared__ float sv[256];
  __shared__ int si[256];
  const int n = p.n;
  const int per = (n + gridDim.x - 1) / gridDim.x;
  const int lo = blockIdx.x * per, hi = min(n, lo + per);
  float bv = -INFINITY;
  int bi = n;
  for (int i = lo + (int)threadIdx.x; i < hi; i += 256) {
    const float v = p.x[i];
    if (better(v, i, bv, bi)) {
      bv = v;
      bi = i;
    }
  }
  block_best(bv, bi, sv, si);
  if (threadIdx.x == 0) {
    p.part_v[blockIdx.x] = bv;
    p.part_i[blockIdx.x] = bi;
  }
}

__global__ __launch_bounds__(256) void argmax_final_kernel(ArgmaxParams p, int parts) {
  __shared__ float sv[256];
  __shared__ int si[256];
  const int n = p.n;
  float bv = -INFINITY;
  int bi = n;
  for (int b = threadIdx.x; b < parts; b += 256) {
    if (better(p.part_v[b], p.part_i[b], bv, bi)) {
      bv = p.part_v[b];
      bi = p.part_i[b];
    }
  }
  block_best(bv, bi, sv, si);
  if (threadIdx.x == 0) {
    // Sequential-scan semantics: a NaN at index 0 is never replaced, and
    // when nothing compares greater than element 0 the answer is 0.
    int best = bi;
    if (best >= n || p.x[0] != p.x[0]) best = 0;
    *p.out = best;
    if (p.seq) {
      const int k = *p.seq_len;
      p.seq[k] = best;
      *p.seq_len = k + 1;
    }
    if (p.pos_inc) *p.pos_inc += 1;
  }
}

}  // namespace

void embed(const int* tok, int T, const uint16_t* table, int d, float* x, hipStream_t s) {
  if (T <= 0) ST_DIE("embed needs T > 0");
  if (d % 8 || (uintptr_t)table % 16 || (uintptr_t)x % 16)
    ST_DIE("embed needs d % 8 == 0 and 16-byte aligned rows (as every GEMV does)");
  hipLaunchKernelGGL(embed8_kernel, dim3(T, (d + 2047) / 2048), dim3(256), 0, s, tok, table, d, x);
  HIP_CHECK(hipGetLastError());
}

void rmsnorm_rows(const float* x, const uint16_t* w, float* y, int rows, int d, float eps,
                  hipStream_t s) {
  if (rows <= 0) ST_DIE("rmsnorm needs rows > 0");
  hipLaunchKernelGGL(rmsnorm_kernel, dim3(rows), dim3(256), 0, s, x, w, y, d, eps);
  HIP_CHECK(hipGetLastError());
}

void residual_norm(const NormParams& p, hipStream_t s) {
  if (p.rows <= 0 || p.d <= 0) ST_DIE("residual_norm needs rows, d > 0");
  if (p.splits > 0 && !p.part) ST_DIE("residual_norm needs the partial sums");
  if (p.routed && (!p.routed_w || p.topk < 1 || (uintptr_t)p.routed % 16))
    ST_DIE("residual_norm: routed sum needs weights, top-k and aligned rows");
  if (p.d % 4 || p.d > 8192) ST_DIE("residual_norm needs d % 4 == 0 and d <= 8192");
  if ((uintptr_t)p.x % 16 || (p.part && (uintptr_t)p.part % 16) || (p.y && (uintptr_t)p.y % 16) ||
      (p.y_hi && (uintptr_t)p.y_hi % 8) || (p.y_lo && (uintptr_t)p.y_lo % 8) || (p.w && (uintptr_t)p.w % 8))
    ST_DIE("residual_norm operands must be aligned");
  const int nv = (p.d / 4 + 255) / 256;
  switch (nv) {
#define RN_CASE(N) \
  case N: hipLaunchKernelGGL(residual_norm_kernel<N>, dim3(p.rows), dim3(256), 0, s, p); break;
    RN_CASE(1) RN_CASE(2) RN_CASE(3) RN_CASE(4) RN_CASE(5) RN_CASE(6) RN_CASE(7) RN_CASE(8)
#undef RN_CASE
    default: ST_DIE("residual_norm: row too long");
  }
  HIP_CHECK(hipGetLastError());
}

bool qk_norm_rope(float* q, int q_heads, float* kcache, int kv_heads, int T, const int* pos,
                  int ctx, int hd, const uint16_t* qn, const uint16_t* kn, float eps,
                  const float* rope, int pair_bound, int pair_offset, int pair_stride,
                  const float* kstage, const PlaneRows* planes, hipStream_t s) {
  if (planes && (!planes->khi || !planes->klo || !planes->vthi || !planes->vtlo || !planes->vcache ||
                 planes->ctx_pad < ctx || planes->kv_bf16 != (kstage != nullptr)))
    ST_DIE("qk_norm_rope: inconsistent plane rows");
  const PlaneRows pl = planes ? *planes : PlaneRows{};
  if (hd > 512 || hd % 2) ST_DIE("head_dim must be even and at most 512");
  if (pair_stride < 1 || pair_bound - pair_stride + pair_offset >= hd)
    ST_DIE("inconsistent RoPE pair geometry");
  const dim3 grid(T, q_heads + kv_heads);
  if ((pair_bound + pair_stride - 1) / pair_stride <= WAVE) {
    const dim3 g4(T, (q_heads + kv_heads + kQkrHeads - 1) / kQkrHeads);
    switch (hd) {
#define QKR_CASE(HD)                                                                                        \
  case HD:                                                                                                 \
    if (planes)                                                                                           \
      hipLaunchKernelGGL((qk_norm_rope_hd_kernel<HD, true>), g4, dim3(kQkrHeads * WAVE), 0, s, q, q_heads, \
                         q_heads + kv_heads, kcache, ctx, pos, qn, kn, eps, rope, pair_bound, pair_offset,  \
                         pair_stride, kstage, pl);                                                        \
    else                                                                                                  \
      hipLaunchKernelGGL((qk_norm_rope_hd_kernel<HD, false>), g4, dim3(kQkrHeads * WAVE), 0, s, q, q_heads, \
                         q_heads + kv_heads, kcache, ctx, pos, qn, kn, eps, rope, pair_bound, pair_offset,  \
                         pair_stride, kstage, pl);                                                        \
    HIP_CHECK(hipGetLastError());                                                                         \
    return planes != nullptr;
      QKR_CASE(16)
      QKR_CASE(32)
      QKR_CASE(64)
      QKR_CASE(128)
#undef QKR_CASE
      default: break;
    }
  }
  hipLaunchKernelGGL(qk_norm_rope_kernel, grid, dim3(64), 0, s, q, q_heads, kcache, ctx, hd, pos, qn, kn, eps,
                     rope, pair_bound, pair_offset, pair_stride, kstage);
  HIP_CHECK(hipGetLastError());
  return false;
}

int argmax_blocks() { return kArgmaxBlocks; }

void argmax(const ArgmaxParams& p, hipStream_t s) {
  if (p.n <= 0) ST_DIE("argmax needs n > 0");
  const int blocks = p.n < kArgmaxBlocks * 256 ? (p.n + 255) / 256 : kArgmaxBlocks;
  hipLaunchKernelGGL(argmax_partial_kernel, dim3(blocks), dim3(256), 0, s, p);
  hipLaunchKernelGGL(argmax_final_kernel, dim3(1), dim3(256), 0, s, p, blocks);
  HIP_CHECK(hipGetLastError());
}

}  // namespace sg
