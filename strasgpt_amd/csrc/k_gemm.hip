// Prefill GEMM on gfx950 MFMA: C[M][N] = A[M][K] x W[N][K]^T with fp32
// activations A and bf16 weights W (both K-contiguous, the Hugging Face
// [out][in] layout needs no repacking).
//
// Precision. The reference keeps activations in fp32 and accumulates
// products in fp32 (source/transformer.c:1097-1167). Weights are exact in
// bf16, so each activation is split into a = hi + lo with hi = bf16(a),
// lo = bf16(a - hi) (a - hi is exact in fp32); both products with a bf16
// weight are exact in the fp32 MFMA accumulator, and the dropped remainder
// is below 2^-17 |a|: fp32-level agreement with the reference for two
// MFMAs per tile (GEMM_SPLIT2). GEMM_BF16 keeps only hi.
//
// Tiling. 256 threads (4 wavefronts as 2x2) per BM x BN tile, K steps of
// 32 staged through double-buffered LDS (A as bf16 hi/lo, W as bf16,
// rows padded to 80 bytes), v_mfma_f32_16x16x32_bf16 on 16x16 sub-tiles.
// Global loads of step k+1 are issued before the MFMAs of step k. The
// SwiGLU variant puts 64 gate rows and the matching 64 up rows of W in one
// B tile so that silu(g) * u is formed in registers.
//
// Algorithmic FLOP per launch: 2 * M * N * K (x2 for the SwiGLU pair).
#include "device_common.h"
#include "hip_check.h"
#include "kernels.h"

namespace sg {

namespace {

constexpr int BK = 32;
constexpr int LDS_STRIDE = BK + 8;  // bf16 elements per LDS row (80 bytes)
constexpr int kThreads = 256;

__device__ __forceinline__ float silu_mul(float g, float u) {
  g *= 1.0f / (1.0f + expf(-g));
  return g * u;
}

__device__ __forceinline__ uint32_t pack2(uint16_t lo, uint16_t hi) {
  return (uint32_t)lo | ((uint32_t)hi << 16);
}

template <int BM, int BN, int EPI, int PREC>
__global__ __launch_bounds__(kThreads, 2) void gemm_kernel(GemmParams p) {
  constexpr bool SPLIT = PREC == GEMM_SPLIT2;
  constexpr bool DUAL = EPI == GEMM_SWIGLU;
  constexpr int WM = BM / 2, WN = BN / 2;   // wavefront tile
  constexpr int MT = WM / 16, NT = WN / 16;  // 16x16 MFMA tiles per wavefront
  constexpr int A_F4 = BM * BK / 4 / kThreads;     // float4 of A per thread
  constexpr int B_U4 = BN * BK / 8 / kThreads;     // uint4 of W per thread
  static_assert(A_F4 >= 1 && B_U4 >= 1, "tile too small for 256 threads");

  __shared__ __attribute__((aligned(16))) uint16_t s_ahi[2][BM * LDS_STRIDE];
  __shared__ __attribute__((aligned(16))) uint16_t s_alo[2][SPLIT ? BM * LDS_STRIDE : 8];
  __shared__ __attribute__((aligned(16))) uint16_t s_b[2][BN * LDS_STRIDE];

  const int tid = threadIdx.x, lane = tid % WAVE, wave = tid / WAVE;
  const int wm = wave / 2, wn = wave % 2;
  const int m0 = blockIdx.y * BM;
  // Output columns covered by this block: BN (plain) or BN/2 gate+up pairs.
  const int n0 = blockIdx.x * (DUAL ? BN / 2 : BN);
  const int M = p.M, N = p.N, K = p.K;

  // W row of each B-tile row r.
  auto b_row = [&](int r) -> int {
    if (!DUAL) return n0 + r;
    return n0 + (r % (BN / 2));
  };
  auto b_src = [&](int r) -> const uint16_t* {
    if (!DUAL) return p.w;
    return r < BN / 2 ? p.w : p.w2;
  };

  float4 ra[A_F4];
  uint4 rb[B_U4];

  auto load_global = [&](int k0) {
#pragma unroll
    for (int i = 0; i < A_F4; i++) {
      const int idx = tid + i * kThreads;
      const int r = idx / (BK / 4), c = (idx % (BK / 4)) * 4;
      const int m = m0 + r;
      ra[i] = m < M ? *(const float4*)(p.a + (size_t)m * p.lda + k0 + c)
                    : make_float4(0.f, 0.f, 0.f, 0.f);
    }
#pragma unroll
    for (int i = 0; i < B_U4; i++) {
      const int idx = tid + i * kThreads;
      const int r = idx / (BK / 8), c = (idx % (BK / 8)) * 8;
      const int n = b_row(r);
      rb[i] = n < N ? *(const uint4*)(b_src(r) + (size_t)n * K + k0 + c)
                    : make_uint4(0u, 0u, 0u, 0u);
    }
  };

  auto store_lds = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_F4; i++) {
      const int idx = tid + i * kThreads;
      const int r = idx / (BK / 4), c = (idx % (BK / 4)) * 4;
      const float v[4] = {ra[i].x, ra[i].y, ra[i].z, ra[i].w};
      uint16_t hi[4], lo[4];
#pragma unroll
      for (int j = 0; j < 4; j++) {
        hi[j] = f32_to_bf16_rne(v[j]);
        lo[j] = SPLIT ? f32_to_bf16_rne(v[j] - bf16_to_f32(hi[j])) : 0;
      }
      *(uint2*)&s_ahi[buf][r * LDS_STRIDE + c] = make_uint2(pack2(hi[0], hi[1]), pack2(hi[2], hi[3]));
      if (SPLIT)
        *(uint2*)&s_alo[buf][r * LDS_STRIDE + c] = make_uint2(pack2(lo[0], lo[1]), pack2(lo[2], lo[3]));
    }
#pragma unroll
    for (int i = 0; i < B_U4; i++) {
      const int idx = tid + i * kThreads;
      const int r = idx / (BK / 8), c = (idx % (BK / 8)) * 8;
      *(uint4*)&s_b[buf][r * LDS_STRIDE + c] = rb[i];
    }
  };

  // B-tile row of n-subtile j of this wavefront.
  auto b_tile_row = [&](int j) -> int {
    if (!DUAL) return wn * WN + j * 16;
    // NT/2 gate subtiles then NT/2 up subtiles covering the same columns.
    const int half = NT / 2;
    const int col = wn * (WN / 2) + (j % half) * 16;
    return (j < half ? 0 : BN / 2) + col;
  };

  f32x4 acc[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; i++)
#pragma unroll
    for (int j = 0; j < NT; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int nk = K / BK;
  load_global(0);
  store_lds(0);
  __syncthreads();
  const int fr = lane % 16, fk = (lane / 16) * 8;
  for (int kt = 0; kt < nk; kt++) {
    const int buf = kt & 1;
    if (kt + 1 < nk) load_global((kt + 1) * BK);
    bf16x8 bfrag[NT];
#pragma unroll
    for (int j = 0; j < NT; j++)
      bfrag[j] = *(const bf16x8*)&s_b[buf][(b_tile_row(j) + fr) * LDS_STRIDE + fk];
#pragma unroll
    for (int i = 0; i < MT; i++) {
      const int ar = (wm * WM + i * 16 + fr) * LDS_STRIDE + fk;
      const bf16x8 ahi = *(const bf16x8*)&s_ahi[buf][ar];
#pragma unroll
      for (int j = 0; j < NT; j++)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ahi, bfrag[j], acc[i][j], 0, 0, 0);
      if (SPLIT) {
        const bf16x8 alo = *(const bf16x8*)&s_alo[buf][ar];
#pragma unroll
        for (int j = 0; j < NT; j++)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(alo, bfrag[j], acc[i][j], 0, 0, 0);
      }
    }
    if (kt + 1 < nk) store_lds(buf ^ 1);
    __syncthreads();
  }

  // Epilogue: lane holds C[4*(lane/16) + e][lane % 16] of each 16x16 tile.
  const int P = (EPI == GEMM_QKV) ? *p.pos : 0;
  const int ecol = lane % 16, erow = (lane / 16) * 4;
#pragma unroll
  for (int i = 0; i < MT; i++) {
#pragma unroll
    for (int j = 0; j < (DUAL ? NT / 2 : NT); j++) {
      const int n = DUAL ? n0 + wn * (WN / 2) + j * 16 + ecol : n0 + wn * WN + j * 16 + ecol;
      if (n >= N) continue;
#pragma unroll
      for (int e = 0; e < 4; e++) {
        const int m = m0 + wm * WM + i * 16 + erow + e;
        if (m >= M) continue;
        const float v = acc[i][j][e];
        if (EPI == GEMM_STORE) {
          p.c[(size_t)m * p.ldc + n] = v;
        } else if (EPI == GEMM_RESIDUAL) {
          p.c[(size_t)m * p.ldc + n] += v;
        } else if (EPI == GEMM_SWIGLU) {
          p.c[(size_t)m * p.ldc + n] = silu_mul(v, acc[i][j + NT / 2][e]);
        } else {  // GEMM_QKV
          if (n < p.q_dim) {
            p.q[(size_t)m * p.q_dim + n] = v;
          } else {
            const int kv = n - p.q_dim;
            float* cache = kv < p.kv_dim ? p.kcache : p.vcache;
            const int j2 = kv < p.kv_dim ? kv : kv - p.kv_dim;
            const int head = j2 / p.head_dim, h = j2 % p.head_dim;
            cache[((size_t)head * p.ctx + P + m) * p.head_dim + h] = v;
          }
        }
      }
    }
  }
}

template <int BM, int BN, int EPI, int PREC>
void launch(const GemmParams& p, hipStream_t s) {
  const int cols = EPI == GEMM_SWIGLU ? BN / 2 : BN;
  dim3 grid((p.N + cols - 1) / cols, (p.M + BM - 1) / BM);
  hipLaunchKernelGGL((gemm_kernel<BM, BN, EPI, PREC>), grid, dim3(kThreads), 0, s, p);
}

template <int EPI, int PREC>
void pick_tile(const GemmParams& p, hipStream_t s) {
  // Large tiles when they still give at least one wave of blocks per CU.
  const int cols = EPI == GEMM_SWIGLU ? 64 : 128;
  const long big = (long)((p.N + cols - 1) / cols) * ((p.M + 127) / 128);
  if (big >= 256)
    launch<128, 128, EPI, PREC>(p, s);
  else
    launch<64, 64, EPI, PREC>(p, s);
}

template <int PREC>
void dispatch(const GemmParams& p, int epi, hipStream_t s) {
  switch (epi) {
    case GEMM_STORE: pick_tile<GEMM_STORE, PREC>(p, s); break;
    case GEMM_RESIDUAL: pick_tile<GEMM_RESIDUAL, PREC>(p, s); break;
    case GEMM_QKV: pick_tile<GEMM_QKV, PREC>(p, s); break;
    case GEMM_SWIGLU: pick_tile<GEMM_SWIGLU, PREC>(p, s); break;
    default: ST_DIE("unknown GEMM epilogue");
  }
}

}  // namespace

int gemm_variant_count() { return 2; }

void gemm_variant(const GemmParams& p, int prec, int v, hipStream_t s) {
  if (p.K % BK) ST_DIE("GEMM needs K to be a multiple of 32");
  if (prec == GEMM_SPLIT2) {
    if (v == 0) launch<128, 128, GEMM_STORE, GEMM_SPLIT2>(p, s);
    else launch<64, 64, GEMM_STORE, GEMM_SPLIT2>(p, s);
  } else {
    if (v == 0) launch<128, 128, GEMM_STORE, GEMM_BF16>(p, s);
    else launch<64, 64, GEMM_STORE, GEMM_BF16>(p, s);
  }
  HIP_CHECK(hipGetLastError());
}

void gemm(const GemmParams& p, int epi, int prec, hipStream_t s) {
  if (p.M <= 0 || p.N <= 0) ST_DIE("GEMM needs M, N > 0");
  if (p.K <= 0 || p.K % BK != 0) ST_DIE("GEMM needs K to be a positive multiple of 32");
  if (p.lda % 4 != 0 || ((uintptr_t)p.a % 16) || ((uintptr_t)p.w % 16))
    ST_DIE("GEMM operands must be 16-byte aligned");
  if (epi == GEMM_SWIGLU && (!p.w2 || (uintptr_t)p.w2 % 16)) ST_DIE("GEMM SwiGLU needs an aligned up matrix");
  if (epi == GEMM_QKV && p.N != p.q_dim + 2 * p.kv_dim) ST_DIE("GEMM QKV column count mismatch");
  if (prec == GEMM_SPLIT2) dispatch<GEMM_SPLIT2>(p, epi, s);
  else if (prec == GEMM_BF16) dispatch<GEMM_BF16>(p, epi, s);
  else ST_DIE("unknown GEMM precision");
  HIP_CHECK(hipGetLastError());
}

}  // namespace sg
