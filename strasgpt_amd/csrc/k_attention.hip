// Causal GQA attention over the device fp32 KV cache
// ([kv_heads][ctx][head_dim] per layer), reference
// source/transformer.c:1375-1422: score = (q . k) / sqrtf(hd), softmax
// with max subtraction and expf, out = sum_s p[s] v[s].
//
// Prefill: one block per (64-query tile, q head); key tiles of 64 staged in
// LDS; 4x4 register-blocked fp32 scores, online softmax (running max and
// sum per query row), P kept in LDS for the P.V product.
//
// Decode: split-K over the cached positions ("flash decoding"): one block
// per (64-key chunk, query head) writes (max, sum, partial output); a
// second small kernel combines the chunks of each head (the kernel boundary
// is the only synchronisation: no device-wide fences).
// The block also applies this step's QK RMSNorm + RoPE to q and to the new
// key (read raw from the QKV projection), and one block per KV head writes
// the processed key into the cache.
#include "device_common.h"
#include "hip_check.h"
#include "kernels.h"

namespace sg {

namespace {

constexpr int BQ = 64, BKV = 64;

template <int HD>
__global__ __launch_bounds__(256) void attn_prefill_kernel(AttnParams p) {
  constexpr int LD = HD + 4;
  constexpr int DU = HD / 16;  // output dims per thread
  __shared__ __attribute__((aligned(16))) float qs[BQ * LD];
  __shared__ __attribute__((aligned(16))) float ks[BKV * LD];
  __shared__ __attribute__((aligned(16))) float vs[BKV * LD];
  __shared__ float ps[BQ * (BKV + 4)];

  const int tid = threadIdx.x, ty = tid / 16, tx = tid % 16;
  const int head = blockIdx.y, q0 = blockIdx.x * BQ;
  const int G = p.q_heads / p.kv_heads, kvh = head / G;
  const int P = *p.pos, T = p.T;
  const int qd = p.q_heads * HD;
  const float* kbase = p.kcache + (size_t)kvh * p.ctx * HD;
  const float* vbase = p.vcache + (size_t)kvh * p.ctx * HD;
  const float scale = sqrtf((float)HD);

  for (int i = tid; i < BQ * HD / 4; i += 256) {
    const int r = i / (HD / 4), c = (i % (HD / 4)) * 4;
    const int t = q0 + r;
    float4 v = t < T ? *(const float4*)(p.q + (size_t)t * qd + head * HD + c)
                     : make_float4(0.f, 0.f, 0.f, 0.f);
    *(float4*)&qs[r * LD + c] = v;
  }

  float m[4], l[4], o[4][DU];
#pragma unroll
  for (int i = 0; i < 4; i++) {
    m[i] = -INFINITY;
    l[i] = 0.0f;
#pragma unroll
    for (int u = 0; u < DU; u++) o[i][u] = 0.0f;
  }

  const int kv_end = min(P + q0 + BQ, P + T);  // keys visible to this tile
  for (int kv0 = 0; kv0 < kv_end; kv0 += BKV) {
    __syncthreads();
    for (int i = tid; i < BKV * HD / 4; i += 256) {
      const int r = i / (HD / 4), c = (i % (HD / 4)) * 4;
      const int s = kv0 + r;
      float4 kv = make_float4(0.f, 0.f, 0.f, 0.f), vv = kv;
      if (s < kv_end) {
        kv = *(const float4*)(kbase + (size_t)s * HD + c);
        vv = *(const float4*)(vbase + (size_t)s * HD + c);
      }
      *(float4*)&ks[r * LD + c] = kv;
      *(float4*)&vs[r * LD + c] = vv;
    }
    __syncthreads();

    float sc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int j = 0; j < 4; j++) sc[i][j] = 0.0f;
    for (int h = 0; h < HD; h += 4) {
      float4 qv[4], kv[4];
#pragma unroll
      for (int i = 0; i < 4; i++) qv[i] = *(const float4*)&qs[(ty * 4 + i) * LD + h];
#pragma unroll
      for (int j = 0; j < 4; j++) kv[j] = *(const float4*)&ks[(tx + 16 * j) * LD + h];
#pragma unroll
      for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) {
          float a = sc[i][j];
          a = fmaf(qv[i].x, kv[j].x, a);
          a = fmaf(qv[i].y, kv[j].y, a);
          a = fmaf(qv[i].z, kv[j].z, a);
          a = fmaf(qv[i].w, kv[j].w, a);
          sc[i][j] = a;
        }
    }
    float corr[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
      const int t = q0 + ty * 4 + i;
      float rmax = -INFINITY;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const int s = kv0 + tx + 16 * j;
        sc[i][j] = (s <= P + t && s < kv_end) ? sc[i][j] / scale : -INFINITY;
        rmax = fmaxf(rmax, sc[i][j]);
      }
      rmax = fmaxf(rmax, __shfl_xor(rmax, 8, WAVE));
      rmax = fmaxf(rmax, __shfl_xor(rmax, 4, WAVE));
      rmax = fmaxf(rmax, __shfl_xor(rmax, 2, WAVE));
      rmax = fmaxf(rmax, __shfl_xor(rmax, 1, WAVE));
      const float mnew = fmaxf(m[i], rmax);
      corr[i] = mnew == -INFINITY ? 1.0f : expf(m[i] - mnew);
      float rsum = 0.0f;
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const float pv = mnew == -INFINITY ? 0.0f : expf(sc[i][j] - mnew);
        ps[(ty * 4 + i) * (BKV + 4) + tx + 16 * j] = pv;
        rsum += pv;
      }
      rsum += __shfl_xor(rsum, 8, WAVE);
      rsum += __shfl_xor(rsum, 4, WAVE);
      rsum += __shfl_xor(rsum, 2, WAVE);
      rsum += __shfl_xor(rsum, 1, WAVE);
      l[i] = l[i] * corr[i] + rsum;
      m[i] = mnew;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
      for (int u = 0; u < DU; u++) o[i][u] *= corr[i];
    const int nk = min(BKV, kv_end - kv0);
    for (int c = 0; c < nk; c++) {
      float pv[4];
#pragma unroll
      for (int i = 0; i < 4; i++) pv[i] = ps[(ty * 4 + i) * (BKV + 4) + c];
#pragma unroll
      for (int u = 0; u < DU; u++) {
        const float vv = vs[c * LD + tx + 16 * u];
#pragma unroll
        for (int i = 0; i < 4; i++) o[i][u] = fmaf(pv[i], vv, o[i][u]);
      }
    }
  }
  // Output as the bf16 hi/lo planes of the O-projection GEMM's input.
#pragma unroll
  for (int i = 0; i < 4; i++) {
    const int t = q0 + ty * 4 + i;
    if (t >= T) continue;
#pragma unroll
    for (int u = 0; u < DU; u++) {
      const float v = o[i][u] / l[i];
      const size_t idx = (size_t)t * qd + head * HD + tx + 16 * u;
      const uint16_t h = f32_to_bf16_rne(v);
      p.out_hi[idx] = h;
      if (p.out_lo) p.out_lo[idx] = f32_to_bf16_rne(v - bf16_to_f32(h));
    }
  }
}

// RMSNorm (optional) + RoPE of one head vector by one wavefront, result in
// LDS `dst`. Same arithmetic as the reference (source/transformer.c:
// 1293-1323).
template <int HD>
__device__ void norm_rope_wave(const float* src, const uint16_t* nw, float eps,
                               const float* cs, int pb, int po, int pst, float* dst) {
#pragma clang fp contract(off)
  const int lane = threadIdx.x % WAVE;
  float ss = 0.0f;
  for (int e = lane; e < HD; e += WAVE) {
    const float x = src[e];
    dst[e] = x;
    ss = fmaf(x, x, ss);
  }
  ss = wave_sum(ss);
  if (nw) {
    const float s = rms_scale(ss, HD, eps);
    for (int e = lane; e < HD; e += WAVE) dst[e] = (dst[e] * s) * bf16_to_f32(nw[e]);
  }
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  float r0[4], r1[4];
  int hh[4];
  int cnt = 0;
  for (int i = lane; i * pst < pb; i += WAVE) {
    const int h = i * pst;
    const float fr = cs[h], fi = cs[h + po];
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

// One block per (64-key chunk, query head). Every global load of the block
// (this chunk's keys and values, the query row, the step's raw key) is
// issued in one round at kernel start, four lanes per key row (128-bit,
// coalesced): the key quarter stays in registers for the scores, the value
// quarter goes to LDS for P.V. The block holding position P uses the
// processed new key for that row and (for the first query head of its
// group) writes it to the cache.
template <int HD>
__global__ __launch_bounds__(256) void attn_decode_kernel(AttnParams p) {
  constexpr int CH = 64, Q4 = HD / 4, NV = Q4 / 4;  // dims per lane, float4 per lane
  __shared__ __attribute__((aligned(16))) float vs[CH * HD];
  __shared__ __attribute__((aligned(16))) float qs[HD];
  __shared__ __attribute__((aligned(16))) float kn[HD];
  __shared__ float sc[CH];
  __shared__ float red[256 / HD][HD];
  __shared__ float stat[2];

  const int split = blockIdx.x, head = blockIdx.y;
  const int G = p.q_heads / p.kv_heads, kvh = head / G;
  const int P = *p.pos, total = P + 1;
  const int nsplit = (total + CH - 1) / CH;
  if (split >= nsplit) return;
  const int s0 = split * CH, s1 = min(s0 + CH, total), n = s1 - s0;
  const int tid = threadIdx.x, wave = tid / WAVE, lane = tid % WAVE;
  const int j = tid / 4, qt = tid % 4;
  const bool has_new = s1 == total;
  const float* kbase = p.kcache + (size_t)kvh * p.ctx * HD;
  const float* vbase = p.vcache + (size_t)kvh * p.ctx * HD;

  float4 kr[NV], vr[NV];
  const bool row = j < n;
  const bool cached = row && s0 + j != P;
#pragma unroll
  for (int i = 0; i < NV; i++) {
    kr[i] = cached ? *(const float4*)(kbase + (size_t)(s0 + j) * HD + qt * Q4 + 4 * i)
                   : make_float4(0.f, 0.f, 0.f, 0.f);
    vr[i] = row ? *(const float4*)(vbase + (size_t)(s0 + j) * HD + qt * Q4 + 4 * i)
                : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  const float* cs = p.rope + (size_t)P * HD;
  if (wave == 0)
    norm_rope_wave<HD>(p.q + (size_t)head * HD, p.qn, p.eps, cs, p.pair_bound, p.pair_offset,
                       p.pair_stride, qs);
  if (wave == 1 && has_new)
    norm_rope_wave<HD>(p.kraw + (size_t)kvh * HD, p.kn, p.eps, cs, p.pair_bound,
                       p.pair_offset, p.pair_stride, kn);
#pragma unroll
  for (int i = 0; i < NV; i++) *(float4*)&vs[j * HD + qt * Q4 + 4 * i] = vr[i];
  __syncthreads();
  if (has_new && head % G == 0) {
    for (int e = tid; e < HD; e += 256) p.kcache_w[((size_t)kvh * p.ctx + P) * HD + e] = kn[e];
  }
  if (row && !cached) {
#pragma unroll
    for (int i = 0; i < NV; i++) kr[i] = *(const float4*)&kn[qt * Q4 + 4 * i];
  }
  float a = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; i++) {
    const float4 q = *(const float4*)&qs[qt * Q4 + 4 * i];
    a = fmaf(q.x, kr[i].x, a);
    a = fmaf(q.y, kr[i].y, a);
    a = fmaf(q.z, kr[i].z, a);
    a = fmaf(q.w, kr[i].w, a);
  }
  a = group_sum<4>(a);
  if (qt == 0 && row) sc[j] = a / sqrtf((float)HD);
  __syncthreads();
  if (wave == 0) {
    const float v = lane < n ? sc[lane] : -INFINITY;
    const float mx = wave_max(v);
    const float e = lane < n ? expf(v - mx) : 0.0f;
    if (lane < n) sc[lane] = e;
    const float sum = wave_sum(e);
    if (lane == 0) {
      stat[0] = mx;
      stat[1] = sum;
    }
  }
  __syncthreads();
  constexpr int KG = 256 / HD;
  const int d = tid % HD, kg = tid / HD;
  {
    float acc = 0.0f;
#pragma unroll 8
    for (int jj = kg; jj < n; jj += KG) acc = fmaf(sc[jj], vs[jj * HD + d], acc);
    red[kg][d] = acc;
  }
  __syncthreads();
  float* part = p.partial + ((size_t)head * p.splits + split) * (HD + 2);
  if (tid < HD) {
    float acc = 0.0f;
#pragma unroll
    for (int k = 0; k < KG; k++) acc += red[k][tid];
    part[2 + tid] = acc;
  }
  if (tid == 0) {
    part[0] = stat[0];
    part[1] = stat[1];
  }
}

// Combines the per-chunk (max, sum, partial output) of one head:
// M = max m_i, out = sum_i o_i e^(m_i - M) / sum_i l_i e^(m_i - M).
template <int HD>
__global__ __launch_bounds__(HD) void attn_decode_combine_kernel(AttnParams p) {
  __shared__ float wts[1024];
  __shared__ float red[HD / WAVE > 0 ? HD / WAVE : 1];
  const int head = blockIdx.x, d = threadIdx.x;
  const int nsplit = (*p.pos + 1 + 63) / 64;
  const float* pb = p.partial + (size_t)head * p.splits * (HD + 2);
  // chunk maxima in parallel, then M = max, weights e^(m_i - M)
  float mx = -INFINITY;
  for (int i = d; i < nsplit; i += HD) {
    wts[i] = pb[(size_t)i * (HD + 2)];
    mx = fmaxf(mx, wts[i]);
  }
  mx = wave_max(mx);
  if (HD > WAVE) {
    if (d % WAVE == 0) red[d / WAVE] = mx;
    __syncthreads();
    for (int w = 0; w < HD / WAVE; w++) mx = fmaxf(mx, red[w]);
  }
  __syncthreads();
  for (int i = d; i < nsplit; i += HD) wts[i] = expf(wts[i] - mx);
  __syncthreads();
  float L = 0.0f, o = 0.0f;
#pragma unroll 4
  for (int i = 0; i < nsplit; i++) {
    const float* q = pb + (size_t)i * (HD + 2);
    L = fmaf(q[1], wts[i], L);
    o = fmaf(q[2 + d], wts[i], o);
  }
  p.out[(size_t)head * HD + d] = o / L;
}

}  // namespace

int attention_decode_splits(int ctx, int chunk) { return (ctx + chunk - 1) / chunk; }

void attention_prefill(const AttnParams& p, hipStream_t s) {
  if (p.T <= 0 || p.q_heads % p.kv_heads) ST_DIE("bad attention shape");
  if (!p.out_hi) ST_DIE("prefill attention writes bf16 planes");
  dim3 grid((p.T + BQ - 1) / BQ, p.q_heads);
  switch (p.hd) {
    case 16: hipLaunchKernelGGL(attn_prefill_kernel<16>, grid, dim3(256), 0, s, p); break;
    case 32: hipLaunchKernelGGL(attn_prefill_kernel<32>, grid, dim3(256), 0, s, p); break;
    case 64: hipLaunchKernelGGL(attn_prefill_kernel<64>, grid, dim3(256), 0, s, p); break;
    case 128: hipLaunchKernelGGL(attn_prefill_kernel<128>, grid, dim3(256), 0, s, p); break;
    default: ST_DIE("attention supports head_dim 16, 32, 64 or 128");
  }
  HIP_CHECK(hipGetLastError());
}

void attention_decode(const AttnParams& p, hipStream_t s) {
  if (p.q_heads % p.kv_heads) ST_DIE("bad attention shape");
  if (p.chunk != 64) ST_DIE("decode attention chunk must be 64");
  if (p.splits != attention_decode_splits(p.ctx, p.chunk)) ST_DIE("decode split count mismatch");
  if (p.splits > 1024) ST_DIE("decode attention supports contexts up to 65536");
  dim3 grid(p.splits, p.q_heads);
  switch (p.hd) {
#define DECODE_CASE(HD)                                                                 \
  case HD:                                                                              \
    hipLaunchKernelGGL(attn_decode_kernel<HD>, grid, dim3(256), 0, s, p);               \
    hipLaunchKernelGGL(attn_decode_combine_kernel<HD>, dim3(p.q_heads), dim3(HD), 0, s, p); \
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
