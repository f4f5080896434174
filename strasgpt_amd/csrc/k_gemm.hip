// Prefill GEMM on gfx950 MFMA: C[M][N] = A[M][K] x W[N][K]^T, bf16
// weights W in the Hugging Face [out][in] layout (no repacking).
//
// Precision. The reference keeps activations in fp32 and accumulates
// products in fp32 (source/transformer.c:1097-1167). Weights are exact in
// bf16, so the producer of each activation matrix stores it split into two
// bf16 planes, a = hi + lo with hi = bf16(a), lo = bf16(a - hi) (a - hi is
// exact in fp32). Both products with a bf16 weight are exact in the fp32
// MFMA accumulator and the dropped remainder is below 2^-17 |a|: fp32-level
// agreement with the reference for two MFMAs per tile (GEMM_SPLIT2).
// GEMM_BF16 uses the hi plane only.
//
// Tiling. 256 threads = 4 wavefronts (2 x 2), block tile BM x BN, K steps
// of 32 streamed through an NS-stage LDS ring filled by asynchronous
// global-to-LDS loads (global_load_lds_dwordx4): NS - 1 K steps are in
// flight while one is multiplied, one barrier per K step, no register
// staging; v_mfma_f32_16x16x32_bf16 on 16x16 sub-tiles. Tiles are
// numbered so that the blocks sharing one column block of W land on the
// same XCD (dispatch is round-robin over the 8 XCDs): W is fetched from
// HBM once per XCD L2. Split-K (grid.z) writes fp32 partial tiles that the
// next kernel (RMSNorm with residual, k_elementwise.hip) sums in order.
//
// Algorithmic FLOP per launch: 2 * M * N * K (x2 for the SwiGLU pair).
#include <cstdlib>
#include <cstring>

#include "device_common.h"
#include "hip_check.h"
#include "kernels.h"

namespace sg {

namespace {

constexpr int BK = 32;
constexpr int kThreads = 256;
constexpr int kXcds = 8;

__device__ __forceinline__ void store_split(uint16_t* hi, uint16_t* lo, size_t i, float v,
                                            bool split) {
  const uint16_t h = f32_to_bf16_rne(v);
  hi[i] = h;
  if (split) lo[i] = f32_to_bf16_rne(v - bf16_to_f32(h));
}

// Block -> (m tile, n tile). Blocks are dispatched round-robin over the
// XCDs; renumber so that each XCD receives a contiguous range of tiles, and
// walk m fastest so that consecutive tiles share W columns.
__device__ __forceinline__ void tile_of(int mt, int nt, int& m_tile, int& n_tile) {
  const int b = blockIdx.x, total = mt * nt;
  int t = b;
  if (total % kXcds == 0) t = (b % kXcds) * (total / kXcds) + b / kXcds;
  m_tile = t % mt;
  n_tile = t / mt;
}

// Waits until at most n vector-memory operations of this wavefront are in
// flight (n is a multiple of the loads issued per stage, at most 31).
__device__ __forceinline__ void wait_vmcnt(int n) {
  // s_waitcnt encoding (gfx9): vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] << 14
#define SG_WAIT(N) __builtin_amdgcn_s_waitcnt(((N) & 15) | (7 << 4) | (15 << 8) | (((N) >> 4) << 14))
  switch (n) {
    case 0: SG_WAIT(0); break;
    case 2: SG_WAIT(2); break;
    case 3: SG_WAIT(3); break;
    case 4: SG_WAIT(4); break;
    case 6: SG_WAIT(6); break;
    case 8: SG_WAIT(8); break;
    case 9: SG_WAIT(9); break;
    case 12: SG_WAIT(12); break;
    case 16: SG_WAIT(16); break;
    case 18: SG_WAIT(18); break;
    case 24: SG_WAIT(24); break;
    default: SG_WAIT(0); break;
  }
#undef SG_WAIT
}

typedef __attribute__((address_space(3))) void* lds_ptr;

// One K step of 32 per stage. LDS rows are 64 bytes (32 bf16) with the four
// 16-byte chunks of row r stored at chunk c ^ swz(r), swz(r) = ((r >> 1) & 3)
// ^ ((r >> 3) & 1) (a function of r mod 16, so the 16-row load groups and
// the fragment reads agree): the 16-byte fragment reads of 8 consecutive
// lanes (rows r..r+7, one chunk) cover all 32 banks once, and those of 16
// consecutive lanes cover 64 banks once. Stages are filled by global_load_lds_dwordx4: one
// wavefront instruction writes 1 KiB = 16 rows, lane i landing at row i/4,
// physical chunk i%4, so lane i fetches the logical chunk that belongs there.
template <int BM, int BN, int NS, int EPI, int PREC, bool PIPE = false>
__global__ __launch_bounds__(kThreads, PIPE ? 2 : 1) void gemm_kernel(GemmParams p) {
  constexpr bool SPLIT = PREC == GEMM_SPLIT2;
  constexpr bool DUAL = EPI == GEMM_SWIGLU;
  constexpr int KS = 32;                       // K per stage
  constexpr int WM = BM / 2, WN = BN / 2;      // wavefront tile
  constexpr int MT = WM / 16, NT = WN / 16;    // 16x16 MFMA tiles per wavefront
  constexpr int A_ROWS = BM * (SPLIT ? 2 : 1);
  constexpr int ROWS = A_ROWS + BN;            // 64-byte rows per stage
  constexpr int GROUPS = ROWS / 16;            // 1 KiB load instructions per stage
  constexpr int PER_WAVE = GROUPS / (kThreads / WAVE);
  static_assert(GROUPS % (kThreads / WAVE) == 0, "stage loads must split evenly over waves");
  static_assert(!DUAL || NT % 2 == 0, "SwiGLU tiles pair gate and up sub-tiles");
  constexpr int STAGE = ROWS * 64;             // bytes

  extern __shared__ __attribute__((aligned(1024))) unsigned char smem[];

  const int tid = threadIdx.x, lane = tid % WAVE, wave = tid / WAVE;
  const int wm = wave / 2, wn = wave % 2;
  const int cols = DUAL ? BN / 2 : BN;
  const int mtiles = (p.M + BM - 1) / BM, ntiles = (p.N + cols - 1) / cols;
  int m_tile, n_tile;
  tile_of(mtiles, ntiles, m_tile, n_tile);
  const int m0 = m_tile * BM, n0 = n_tile * cols;
  const int M = p.M, N = p.N, K = p.K;
  const int ksplit = gridDim.z, kper = ((K + KS - 1) / KS + ksplit - 1) / ksplit * KS;
  const int kbeg = blockIdx.z * kper, kend = min(K, kbeg + kper);
  const int nk = kend > kbeg ? (kend - kbeg) / KS : 0;

  // Per-lane global source of each load group this wavefront issues.
  const uint16_t* src[PER_WAVE];
  {
    const int r16 = lane / 4, phys = lane % 4;
#pragma unroll
    for (int i = 0; i < PER_WAVE; i++) {
      const int g = wave * PER_WAVE + i;
      const int row = g * 16 + r16;  // row in the stage
      const int c = phys ^ (((r16 >> 1) & 3) ^ ((r16 >> 3) & 1));
      if (row < A_ROWS) {
        const int r = row % BM;
        const int m = min(m0 + r, M - 1);  // rows past M load row M-1, never stored
        const uint16_t* base = (SPLIT && row >= BM) ? p.a_lo : p.a_hi;
        src[i] = base + (size_t)m * p.lda + c * 8;
      } else {
        const int r = row - A_ROWS;
        const int nn = min(DUAL ? n0 + (r % (BN / 2)) : n0 + r, N - 1);
        const uint16_t* base = (DUAL && r >= BN / 2) ? p.w2 : p.w;
        src[i] = base + (size_t)nn * K + c * 8;
      }
    }
  }
  auto issue = [&](int t) {
    unsigned char* st = smem + (t % NS) * STAGE;
    const int k0 = kbeg + t * KS;
#pragma unroll
    for (int i = 0; i < PER_WAVE; i++) {
      const int g = wave * PER_WAVE + i;
      __builtin_amdgcn_global_load_lds((const void*)(src[i] + k0), (lds_ptr)(st + g * 1024), 16, 0, 0);
    }
  };
  auto frag = [&](const unsigned char* base, int r) -> bf16x8 {
    const int c = lane / 16;
    return *(const bf16x8*)(base + r * 64 + ((c ^ (((r >> 1) & 3) ^ ((r >> 3) & 1))) << 4));
  };
  auto b_tile_row = [&](int j) -> int {
    if (!DUAL) return wn * WN + j * 16;
    const int half = NT / 2;
    return (j < half ? 0 : BN / 2) + wn * (WN / 2) + (j % half) * 16;
  };

  f32x4 acc[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; i++)
#pragma unroll
    for (int j = 0; j < NT; j++) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

#pragma unroll
  for (int t = 0; t < NS - 1; t++)
    if (t < nk) issue(t);
  const int fr = lane % 16;
  if constexpr (PIPE) {
    // Fragments of K step kt+1 are read from LDS while the MFMAs of step kt
    // run (two register sets, alternating without copies). At step kt:
    // wait for stage kt+1, barrier (every wave has read stage kt-1's
    // fragments, so its buffer is free), issue stage kt+NS-1, read step
    // kt+1's fragments, multiply step kt.
    static_assert(NS >= 3, "fragment pipelining needs three stages");
    struct Frags {
      bf16x8 b[NT];
      bf16x8 ahi[MT];
      bf16x8 alo[SPLIT ? MT : 1];
    };
    auto read_frags = [&](int kt, Frags& F) {
      const unsigned char* st = smem + (kt % NS) * STAGE;
#pragma unroll
      for (int j = 0; j < NT; j++) F.b[j] = frag(st + A_ROWS * 64, b_tile_row(j) + fr);
#pragma unroll
      for (int i = 0; i < MT; i++) {
        const int r = wm * WM + i * 16 + fr;
        F.ahi[i] = frag(st, r);
        if (SPLIT) F.alo[i] = frag(st + BM * 64, r);
      }
    };
    auto mma = [&](const Frags& F) {
#pragma unroll
      for (int i = 0; i < MT; i++) {
#pragma unroll
        for (int j = 0; j < NT; j++)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(F.ahi[i], F.b[j], acc[i][j], 0, 0, 0);
        if (SPLIT) {
#pragma unroll
          for (int j = 0; j < NT; j++)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(F.alo[i], F.b[j], acc[i][j], 0, 0, 0);
        }
      }
    };
    auto step = [&](int kt, const Frags& cur, Frags& nxt) {
      if (kt + 1 < nk) {
        // stages issued so far: 0 .. min(kt + NS - 2, nk - 1); keep those
        // after kt + 1 in flight
        const int ahead = min(kt + NS - 2, nk - 1) - (kt + 1);
        wait_vmcnt(ahead * PER_WAVE);
        __builtin_amdgcn_s_barrier();
        if (kt + NS - 1 < nk) issue(kt + NS - 1);
        read_frags(kt + 1, nxt);
      }
      mma(cur);
    };
    Frags f0, f1;
    if (nk > 0) {
      wait_vmcnt(min(NS - 2, nk - 1) * PER_WAVE);
      __builtin_amdgcn_s_barrier();
      read_frags(0, f0);
    }
    for (int kt = 0; kt < nk; kt += 2) {
      step(kt, f0, f1);
      if (kt + 1 >= nk) break;
      step(kt + 1, f1, f0);
    }
  } else
  for (int kt = 0; kt < nk; kt++) {
    const int ahead = min(NS - 2, nk - 1 - kt);  // stages still allowed in flight
    wait_vmcnt(ahead * PER_WAVE);
    __builtin_amdgcn_s_barrier();
    if (kt + NS - 1 < nk) issue(kt + NS - 1);
    const unsigned char* st = smem + (kt % NS) * STAGE;
    bf16x8 bfrag[NT];
#pragma unroll
    for (int j = 0; j < NT; j++) bfrag[j] = frag(st + A_ROWS * 64, b_tile_row(j) + fr);
#pragma unroll
    for (int i = 0; i < MT; i++) {
      const int r = wm * WM + i * 16 + fr;
      const bf16x8 ahi = frag(st, r);
#pragma unroll
      for (int j = 0; j < NT; j++)
        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ahi, bfrag[j], acc[i][j], 0, 0, 0);
      if (SPLIT) {
        const bf16x8 alo = frag(st + BM * 64, r);
#pragma unroll
        for (int j = 0; j < NT; j++)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(alo, bfrag[j], acc[i][j], 0, 0, 0);
      }
    }
  }

  // Epilogue: lane holds C[4*(lane/16) + e][lane % 16] of each 16x16 tile.
  const int P = (EPI == GEMM_QKV) ? *p.pos : 0;
  const int ecol = lane % 16, erow = (lane / 16) * 4;
  const bool out_split = p.c_lo != nullptr;
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
        } else if (EPI == GEMM_PARTIAL) {
          p.c[((size_t)blockIdx.z * M + m) * p.ldc + n] = v;
        } else if (EPI == GEMM_SWIGLU) {
          // the output is the next GEMM's A operand: store it split
          store_split(p.c_hi, p.c_lo, (size_t)m * p.ldc + n, silu_mul(v, acc[i][j + NT / 2][e]),
                      out_split);
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

template <int BM, int BN, int NS, int EPI, int PREC, bool PIPE = false>
void launch(const GemmParams& p, int splits, hipStream_t s) {
  const int cols = EPI == GEMM_SWIGLU ? BN / 2 : BN;
  const int tiles = ((p.N + cols - 1) / cols) * ((p.M + BM - 1) / BM);
  constexpr int rows = BM * (PREC == GEMM_SPLIT2 ? 2 : 1) + BN;
  constexpr size_t shm = (size_t)NS * rows * 64;
  static_assert(shm <= 160 * 1024, "GEMM stages exceed LDS");
  static bool attr = false;
  if (!attr) {
    HIP_CHECK(hipFuncSetAttribute((const void*)gemm_kernel<BM, BN, NS, EPI, PREC, PIPE>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm));
    attr = true;
  }
  hipLaunchKernelGGL((gemm_kernel<BM, BN, NS, EPI, PREC, PIPE>), dim3(tiles, 1, splits), dim3(kThreads),
                     shm, s, p);
}

// Tile shape forced by STRASGPT_GEMM_TILE ("128x256", "128x128", "64x128",
// "64x64"), for tests that run every shape on small models; 0 = by size.
int forced_tile() {
  const char* v = getenv("STRASGPT_GEMM_TILE");
  if (!v || !*v) return 0;
  if (!strcmp(v, "128x256")) return 4;
  if (!strcmp(v, "128x128")) return 3;
  if (!strcmp(v, "64x128")) return 2;
  if (!strcmp(v, "64x64")) return 1;
  ST_DIE("STRASGPT_GEMM_TILE must be 128x256, 128x128, 64x128 or 64x64");
}

template <int EPI, int PREC>
void dispatch_tile(const GemmParams& p, int splits, hipStream_t s) {
  // Measured on MI355X: with two blocks of 128 x 256 tiles per CU or more
  // (M >= 2048 prefill shapes), those tiles (wavefront tile 64 x 128: fewer
  // LDS bytes per MFMA; 64 KiB of LDS, two blocks per CU) reach ~45% of the
  // MFMA rate against ~30% for 128 x 128; with two blocks of 128 x 128 per
  // CU, 128 x 128 with a 2-stage ring (48 KiB: three blocks per CU) beats
  // deeper rings; from about one block per CU, 64 x 128 with 4 stages;
  // below that 64 x 64.
  const int cols = EPI == GEMM_SWIGLU ? 64 : 128;
  const long big = (long)((p.N + cols - 1) / cols) * ((p.M + 127) / 128) * splits;
  const long wide = (long)((p.N + 2 * cols - 1) / (2 * cols)) * ((p.M + 127) / 128) * splits;
  int shape = forced_tile();
  if (!shape) shape = wide >= 512 ? 4 : big >= 512 ? 3 : big >= 192 ? 2 : 1;
  switch (shape) {
    case 4: launch<128, 256, 2, EPI, PREC>(p, splits, s); break;
    case 3: launch<128, 128, 2, EPI, PREC>(p, splits, s); break;
    case 2: launch<64, 128, 4, EPI, PREC>(p, splits, s); break;
    default: launch<64, 64, 4, EPI, PREC>(p, splits, s); break;
  }
}

template <int PREC>
void dispatch(const GemmParams& p, int epi, int splits, hipStream_t s) {
  switch (epi) {
    case GEMM_STORE: dispatch_tile<GEMM_STORE, PREC>(p, splits, s); break;
    case GEMM_RESIDUAL: dispatch_tile<GEMM_RESIDUAL, PREC>(p, splits, s); break;
    case GEMM_QKV: dispatch_tile<GEMM_QKV, PREC>(p, splits, s); break;
    case GEMM_SWIGLU: dispatch_tile<GEMM_SWIGLU, PREC>(p, splits, s); break;
    case GEMM_PARTIAL: dispatch_tile<GEMM_PARTIAL, PREC>(p, splits, s); break;
    default: ST_DIE("unknown GEMM epilogue");
  }
}

void check(const GemmParams& p, int epi, int prec, int splits) {
  if (p.M <= 0 || p.N <= 0) ST_DIE("GEMM needs M, N > 0");
  if (p.K <= 0 || p.K % 32 != 0) ST_DIE("GEMM needs K to be a positive multiple of 32");
  if (p.lda % 8 != 0 || ((uintptr_t)p.a_hi % 16) || ((uintptr_t)p.w % 16))
    ST_DIE("GEMM operands must be 16-byte aligned");
  if (p.K % 8 != 0) ST_DIE("GEMM needs K to be a multiple of 8");
  if (prec == GEMM_SPLIT2 && (!p.a_lo || (uintptr_t)p.a_lo % 16)) ST_DIE("GEMM bf16x2 needs the lo plane");
  if (epi == GEMM_SWIGLU && (!p.w2 || (uintptr_t)p.w2 % 16 || !p.c_hi)) ST_DIE("GEMM SwiGLU operands");
  if (epi == GEMM_QKV && p.N != p.q_dim + 2 * p.kv_dim) ST_DIE("GEMM QKV column count mismatch");
  if (splits < 1 || splits > 16 || (splits > 1 && epi != GEMM_PARTIAL))
    ST_DIE("GEMM split-K is only available with the partial-sum epilogue");
}

}  // namespace

int gemm_splits(int M, int N, int K) {
  // Enough blocks for the 256 CUs on the N = embedding_dim projections;
  // long reductions (K >= 16384: a 1024-step K loop and more) split until
  // there are about four 128 x 128 tiles per CU.
  const long tiles = (long)((N + 127) / 128) * ((M + 127) / 128);
  const long want = K >= 16384 ? 1024 : 192;
  if (tiles >= want) return 1;
  int s = (int)((K >= 16384 ? want : 256) + tiles - 1) / (int)tiles;
  while (s > 1 && (K + BK - 1) / BK < 4 * s) s--;  // keep at least 4 K tiles per split
  return s < 1 ? 1 : s;
}

void gemm(const GemmParams& p, int epi, int prec, int splits, hipStream_t s) {
  check(p, epi, prec, splits);
  if (prec == GEMM_SPLIT2) dispatch<GEMM_SPLIT2>(p, epi, splits, s);
  else if (prec == GEMM_BF16) dispatch<GEMM_BF16>(p, epi, splits, s);
  else ST_DIE("unknown GEMM precision");
  HIP_CHECK(hipGetLastError());
}

int gemm_variant_count() { return 14; }

void gemm_variant(const GemmParams& p, int prec, int v, hipStream_t s) {
  check(p, GEMM_STORE, prec, 1);
#define GP(BM, BN, NS)                                                                \
  if (prec == GEMM_SPLIT2) launch<BM, BN, NS, GEMM_STORE, GEMM_SPLIT2, true>(p, 1, s); \
  else launch<BM, BN, NS, GEMM_STORE, GEMM_BF16, true>(p, 1, s);                      \
  break;
#define G(BM, BN, NS)                                                        \
  if (prec == GEMM_SPLIT2) launch<BM, BN, NS, GEMM_STORE, GEMM_SPLIT2>(p, 1, s); \
  else launch<BM, BN, NS, GEMM_STORE, GEMM_BF16>(p, 1, s);                   \
  break;
  switch (v) {
    case 0: G(128, 128, 4)
    case 1: G(128, 128, 3)
    case 2: G(64, 64, 4)
    case 3: G(128, 64, 4)
    case 4: G(64, 128, 4)
    case 5: G(128, 128, 2)
    case 6: G(128, 256, 2)
    case 7: G(128, 256, 3)
    case 8: G(64, 256, 3)
    case 9: GP(128, 128, 3)
    case 10: GP(128, 128, 4)
    case 11: GP(64, 128, 4)
    case 12: GP(128, 256, 3)
    case 13: GP(64, 128, 3)
    default: ST_DIE("unknown GEMM variant");
  }
#undef G
#undef GP
  HIP_CHECK(hipGetLastError());
}

}  // namespace sg
