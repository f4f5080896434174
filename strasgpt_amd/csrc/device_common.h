// Device helpers shared by the gfx950 kernels: bf16 / MXFP4 decoding,
// wavefront (64-lane) reductions, vector types for 128-bit memory access.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#define WAVE 64

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float float2v __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

// bf16 bits are the upper half of the fp32 bits (reference
// include/util.h:33-39): exact.
__device__ __forceinline__ float bf16_lo(uint32_t packed) {
  return __uint_as_float(packed << 16);
}
__device__ __forceinline__ float bf16_hi(uint32_t packed) {
  return __uint_as_float(packed & 0xFFFF0000u);
}
__device__ __forceinline__ float bf16_to_f32(uint16_t w) {
  return __uint_as_float((uint32_t)w << 16);
}

// Round-to-nearest-even fp32 -> bf16 bits (finite inputs).
__device__ __forceinline__ uint16_t f32_to_bf16_rne(float f) {
  uint32_t u = __float_as_uint(f);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// The same rounding for every value: NaNs stay NaN (quieted), infinities
// stay (the KV-cache bf16 format).
__device__ __forceinline__ uint16_t f32_to_bf16_any(float f) {
  uint32_t u = __float_as_uint(f);
  u = (u & 0x7FFFFFFFu) > 0x7F800000u ? u | 0x00400000u : u + 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

// MXFP4 (OCP MX v1.0) E2M1 element: sign bit 3, exponent bits 2..1,
// mantissa bit 0. Magnitudes 0, .5, 1, 1.5, 2, 3, 4, 6 built directly as
// fp32 bit patterns: exponent e >= 1 gives 2^(e-1) * (1 + m/2).
__device__ __forceinline__ float e2m1_value(uint32_t code) {
  const uint32_t e = (code >> 1) & 3u, m = code & 1u;
  float v = e ? __uint_as_float(((126u + e) << 23) | (m << 22)) : (m ? 0.5f : 0.0f);
  return (code & 8u) ? -v : v;
}
__device__ __forceinline__ float e8m0_scale(uint32_t s) {
  // 2^(s-127) as an fp32 bit pattern: s << 23 for 1 <= s <= 254; s = 0
  // gives 2^-127 (subnormal, 0x00400000) and s = 255 NaN (0x7FC00000).
  // Integer arithmetic only (s <= 255): (s - 1) >> 31 is 1 only for s = 0,
  // (s + 1) >> 8 only for s = 255, so the compiler emits no branch (a
  // branch right after the byte load would wait for it).
  return __uint_as_float((s << 23) | (((s - 1u) >> 31) << 22) | (((s + 1u) >> 8) << 22));
}

// 16-byte streaming load of weights that are read once per step.
// Plain accesses through pointers known to address global memory.
__device__ __forceinline__ float gload(const float* p) {
  return *(__attribute__((address_space(1))) const float*)p;
}
__device__ __forceinline__ float4 gload4(const float* p) {
  typedef float f4 __attribute__((ext_vector_type(4)));
  const f4 v = *(__attribute__((address_space(1))) const f4*)p;
  return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint16_t gload(const uint16_t* p) {
  return *(__attribute__((address_space(1))) const uint16_t*)p;
}
__device__ __forceinline__ void gstore(float* p, float v) {
  *(__attribute__((address_space(1))) float*)p = v;
}

// global_load_lds_dwordx4: 16 bytes per lane from g to LDS at l
// (wave-uniform) + 16 * lane, written out in assembly (M0 saved and
// restored around it). Issued through the compiler builtin, an LDS DMA
// makes the compiler turn every later wait on vector memory into
// vmcnt(0) while it is pending (a staging wait meant to leave the loads
// issued after the DMA in flight drains them; a wait for a value loaded
// before the DMA waits for the DMA too). Hidden from the compiler, the DMA
// is ordered by the caller's explicit s_waitcnt before a barrier; the
// compiler's own waits for later loads, which it counts without the older
// DMA, are then exact or longer. (In the MXFP4 expert GEMVs, selecting the
// experts first and then issuing this DMA and the weights measured 0.6%
// slower than the DMA first with the builtin.)
__device__ __forceinline__ void dma16_hidden(const void* g, __attribute__((address_space(3))) void* l) {
  const int base = __builtin_amdgcn_readfirstlane((int)(uintptr_t)l);
  int saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %1, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(g), "s"(base)
      : "memory");
}

typedef __bf16 bf16x2v __attribute__((ext_vector_type(2)));
typedef float f32x2v __attribute__((ext_vector_type(2)));

// (a, b) -> packed bf16 hi pair and lo pair: hi = bf16(x) (round to nearest
// even, v_cvt_pk_bf16_f32), lo = bf16(x - hi) with x - hi exact in fp32.
__device__ __forceinline__ void split2(float a, float b, uint32_t& hi, uint32_t& lo) {
  const bf16x2v h = __builtin_convertvector((f32x2v){a, b}, bf16x2v);
  const uint32_t hb = __builtin_bit_cast(uint32_t, h);
  const float ra = a - __builtin_bit_cast(float, hb << 16);
  const float rb = b - __builtin_bit_cast(float, hb & 0xffff0000u);
  hi = hb;
  lo = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2v){ra, rb}, bf16x2v));
}

// 128-bit non-temporal load from global memory (global, not flat,
// instructions whatever the compiler knows of where `p` came from).
__device__ __forceinline__ uint4 load_nt_u4(const void* p) {
  typedef __attribute__((address_space(1))) const uint4 guint4;
  const guint4* q = (const guint4*)p;
  uint4 r;
  r.x = __builtin_nontemporal_load(&q->x);
  r.y = __builtin_nontemporal_load(&q->y);
  r.z = __builtin_nontemporal_load(&q->z);
  r.w = __builtin_nontemporal_load(&q->w);
  return r;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, WAVE);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, WAVE));
  return v;
}

// Sum / maximum over the 64 lanes of a wave (all lanes active), the same in
// every lane: within each row of 16 lanes by DPP moves (no LDS traffic),
// then the four row results read as scalars.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float x) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(x), CTRL, 0xf, 0xf, false));
}

__device__ __forceinline__ float wave_total(float v) {
  v += dpp_mov<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_mov<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_mov<0x141>(v);  // row_half_mirror
  v += dpp_mov<0x140>(v);  // row_mirror
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (r0 + r1) + (r2 + r3);
}

__device__ __forceinline__ float wave_peak(float v) {
  v = fmaxf(v, dpp_mov<0xB1>(v));
  v = fmaxf(v, dpp_mov<0x4E>(v));
  v = fmaxf(v, dpp_mov<0x141>(v));
  v = fmaxf(v, dpp_mov<0x140>(v));
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// Sum over a power-of-two group of `width` lanes (aligned groups).
template <int WIDTH>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int off = WIDTH / 2; off >= 1; off >>= 1) v += __shfl_xor(v, off, WAVE);
  return v;
}

// Block-wide sum for blockDim.x == NT (multiple of 64); `red` holds
// NT/64 floats of shared memory. Every thread gets the result.
template <int NT>
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wave_sum(v);
  const int w = threadIdx.x / WAVE, l = threadIdx.x % WAVE;
  if (l == 0) red[w] = v;
  __syncthreads();
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < NT / WAVE; i++) s += red[i];
  __syncthreads();
  return s;
}

// acc + dot(8 bf16 weights packed in w, fp32 a[0..3] and b[0..3]), in
// element order.
__device__ __forceinline__ float dot8(uint4 w, const float4& a, const float4& b, float acc) {
  acc = fmaf(bf16_lo(w.x), a.x, acc);
  acc = fmaf(bf16_hi(w.x), a.y, acc);
  acc = fmaf(bf16_lo(w.y), a.z, acc);
  acc = fmaf(bf16_hi(w.y), a.w, acc);
  acc = fmaf(bf16_lo(w.z), b.x, acc);
  acc = fmaf(bf16_hi(w.z), b.y, acc);
  acc = fmaf(bf16_lo(w.w), b.z, acc);
  acc = fmaf(bf16_hi(w.w), b.w, acc);
  return acc;
}

// SwiGLU of one element: silu(g) * u (reference source/transformer.c:
// 1477-1486).
__device__ __forceinline__ float silu_mul(float g, float u) {
  g *= 1.0f / (1.0f + expf(-g));
  return g * u;
}

// RMSNorm scale exactly as the reference computes it from the sum of
// squares (source/transformer.c:990-992): ss/n, then
// (float)(1.0 / sqrtf(ss + eps)).
__device__ __forceinline__ float rms_scale(float ss, int n, float eps) {
  ss /= (float)n;
  return (float)(1.0 / (double)sqrtf(ss + eps));
}

// Compiler-only ordering point: no memory access is moved across it by the
// compiler (no instruction is emitted). The cross-block hand-offs put one
// before the wait that completes a block's partial stores and one after the
// arrival check, so that their order is fixed in the code as well as by
// the wait and the control dependence on the arrival count.
__device__ __forceinline__ void compiler_fence() { asm volatile("" ::: "memory"); }

// Agent-coherent scalar access: relaxed atomics at device scope, which
// bypass the per-XCD L2 for data exchanged between blocks of one launch.
// A store is visible to another block's cload once the storing wave has
// waited for its vector memory operations to complete.
__device__ __forceinline__ float cload(const float* p) {
  return __hip_atomic_load((const __attribute__((address_space(1))) float*)p, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ int cload(const int* p) {
  return __hip_atomic_load((const __attribute__((address_space(1))) int*)p, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
}
// Two consecutive floats (8-byte aligned) in one agent-coherent load.
__device__ __forceinline__ float2 cload2(const float* p) {
  const unsigned long long u = __hip_atomic_load((const __attribute__((address_space(1))) unsigned long long*)p,
                                                 __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  return make_float2(__uint_as_float((unsigned)u), __uint_as_float((unsigned)(u >> 32)));
}
__device__ __forceinline__ void cstore(float* p, float v) {
  __hip_atomic_store((__attribute__((address_space(1))) float*)p, v, __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void cstore(int* p, int v) {
  __hip_atomic_store((__attribute__((address_space(1))) int*)p, v, __ATOMIC_RELAXED,
                     __HIP_MEMORY_SCOPE_AGENT);
}
