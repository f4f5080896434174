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
#include <algorithm>
#include <cstdlib>
#include <cstring>

#include "device_common.h"
#include "hip_check.h"
#include "kernels.h"

namespace sg {

namespace {

constexpr int BK = 32;
constexpr int kXcds = 8;

__device__ __forceinline__ void store_split(uint16_t* hi, uint16_t* lo, size_t i, float v,
                                            bool split) {
  const uint16_t h = f32_to_bf16_rne(v);
  hi[i] = h;
  if (split) lo[i] = f32_to_bf16_rne(v - bf16_to_f32(h));
}

// Block -> (m tile, n tile). Blocks are dispatched round-robin over the
// XCDs; renumber so that each XCD receives a contiguous range of tiles.
// Order 0 (the 16x16x32 kernels): tiles in groups of kGroupM row tiles,
// m fastest within a group, then n; the blocks resident on one XCD at a
// time cover about 8 row tiles x 4 column tiles, so each A and W tile
// fetched into that XCD's L2 serves several blocks (with every row tile in
// flight at once, m fastest over all of M, each A tile would be fetched
// once per block).
// The 256 x 256 kernel (order 3 by default; STRASGPT_GEMM_ORDER forces 0-3
// for measurements and tests): the tile grid is cut into 2 x 4 rectangles,
// one per XCD, each walked m fastest within groups of 4 row tiles, so the
// 32 blocks resident on an XCD cover 4 row tiles x 8 column tiles. Per
// K step they then fetch 4 A tiles (32 KiB each as hi + lo planes) and 8 W
// tiles (16 KiB) instead of 8 and 4: 256 instead of 320 KiB. Measured on
// the Mistral-Small-24B shape at 2048 tokens: down (split-K, 8 x 20 tiles
// per split) 1296 -> 1061 us, gate/up 2073 -> 2013 us, prefill +7.7%;
// neutral on Llama-3.1-8B at 8192 tokens and Qwen3-4B at 512. Order 1
// (whole row panels per XCD) and order 2 (rectangles walked m fastest over
// the whole rectangle: 16 x 2 at 8192 tokens) measured no better than 0.
constexpr int kGroupM = 8;
__device__ __forceinline__ void tile_of(int mt, int nt, int& m_tile, int& n_tile, int order = 0) {
  const int b = blockIdx.x, total = mt * nt;
  int t = b;
  if (total % kXcds == 0) t = (b % kXcds) * (total / kXcds) + b / kXcds;
  if (order == 1 && total % kXcds == 0) {
    // row panels: each XCD takes whole rows of tiles, n fastest (one A
    // panel shared by every block of the XCD)
    m_tile = t / nt;
    n_tile = t % nt;
    return;
  }
  if (order >= 2 && total % kXcds == 0 && mt % 2 == 0 && nt % 4 == 0) {
    // the tile grid cut into 2 x 4 rectangles, one per XCD, each walked
    // m fastest (order 2), or m fastest within groups of 4 row tiles
    // (order 3)
    const int rm = mt / 2, rn = nt / 4, x = t / (rm * rn), in = t % (rm * rn);
    const int gm = order == 3 ? 4 : rm, g = in / (gm * rn), rows = min(gm, rm - g * gm);
    const int local = in - g * gm * rn;
    m_tile = (x / 4) * rm + g * gm + local % rows;
    n_tile = (x % 4) * rn + local / rows;
    return;
  }
  const int group = t / (kGroupM * nt), first = group * kGroupM;
  const int rows = min(kGroupM, mt - first), in = t - group * kGroupM * nt;
  m_tile = first + in % rows;
  n_tile = in / rows;
}

// Waits until at most n vector-memory operations of this wavefront are in
// flight (n is a multiple of the loads issued per stage; counts that are not
// listed wait for everything, which is correct but slower).
__device__ __forceinline__ void wait_vmcnt(int n) {
  // s_waitcnt encoding (gfx9): vmcnt[3:0] | expcnt[6:4] | lgkmcnt[11:8] | vmcnt[5:4] << 14
#define SG_WAIT(N) \
  case N: __builtin_amdgcn_s_waitcnt(((N) & 15) | (7 << 4) | (15 << 8) | (((N) >> 4) << 14)); break;
  switch (n) {
    SG_WAIT(2) SG_WAIT(3) SG_WAIT(4) SG_WAIT(5) SG_WAIT(6) SG_WAIT(8) SG_WAIT(9) SG_WAIT(10)
    SG_WAIT(12) SG_WAIT(15) SG_WAIT(16) SG_WAIT(18) SG_WAIT(20) SG_WAIT(24) SG_WAIT(30)
    SG_WAIT(32) SG_WAIT(36) SG_WAIT(40) SG_WAIT(48)
    default: __builtin_amdgcn_s_waitcnt((7 << 4) | (15 << 8)); break;
  }
#undef SG_WAIT
}

typedef __attribute__((address_space(3))) void* lds_ptr;

// One K step of 32 per stage. LDS rows are 64 bytes (32 bf16) with the four
// 16-byte chunks of row r stored at chunk c ^ swz(r), swz(r) = (-(r >> 2)) & 3
// (a function of r mod 16, so the 16-row load groups and the fragment reads
// agree). A fragment read is ds_read_b128 with lane l reading row l % 16,
// logical chunk l / 16. gfx950 has 64 four-byte banks and serves a 128-bit
// read in four phases of 16 lanes: within each half wavefront, the lane
// quads (l >> 2) & 7 of even bit parity form one phase and those of odd
// parity the other (measured with the bank-conflict counters). Rows r and
// r + 4j share banks for a given chunk, so each phase's four quads must land
// on four different physical chunks; this swizzle does that for both
// parities (a conflict costs a second pass: 8 instead of 4 LDS cycles per
// read). Stages are filled by global_load_lds_dwordx4: one wavefront
// instruction writes 1 KiB = 16 rows, lane i landing at row i/4, physical
// chunk i%4, so lane i fetches the logical chunk that belongs there.
//
// K steps of 64 per stage use 128-byte rows (eight chunks; rows r and r + 2j
// share banks): swz(r) = (r >> 1) & 7 spreads each phase's rows over the
// eight chunks of both bank halves. A 128-byte row segment per DMA lane
// group moves about 1.8x the bytes per cycle of a 64-byte one through the
// CU's texture path (L2-resident microbenchmark), which is what limits the
// 32-deep stages.
template <int KS>
__device__ __forceinline__ int lds_swz(int r) {
  return KS == 32 ? (0 - (r >> 2)) & 3 : (r >> 1) & 7;
}

// OCC: blocks per CU the register allocation must allow (0: one).
// WD = 1: the W tiles get a ring one stage deeper than the A tiles (A is
// re-read by every column block and stays in cache; W streams from HBM once
// per XCD), loads issued so that W has one more K step of latency cover.
// NW: wavefronts per block, arranged NW/2 (rows) x 2 (columns).
template <int BM, int BN, int NS, int EPI, int PREC, int OCC = 0, int KS = 32, int WD = 0, int NW = 4>
__global__ __launch_bounds__(NW * WAVE, OCC ? OCC : 1) void gemm_kernel(GemmParams p) {
  constexpr bool SPLIT = PREC == GEMM_SPLIT2;
  constexpr bool DUAL = EPI == GEMM_SWIGLU;
  static_assert(KS == 32 || KS == 64, "K per stage");
  constexpr int ROWB = KS * 2;                 // bytes per LDS row
  constexpr int CPR = ROWB / 16;               // 16-byte chunks per row
  constexpr int RPI = 1024 / ROWB;             // rows per 1 KiB load instruction
  constexpr int KSUB = KS / 32;                // MFMA k-steps per stage
  constexpr int WGM = NW / 2;                  // wavefront rows
  constexpr int WM = BM / WGM, WN = BN / 2;    // wavefront tile
  constexpr int MT = WM / 16, NT = WN / 16;    // 16x16 MFMA tiles per wavefront
  constexpr int A_ROWS = BM * (SPLIT ? 2 : 1);
  constexpr int ROWS = A_ROWS + BN;            // rows per stage
  constexpr int GROUPS = ROWS / RPI;           // 1 KiB load instructions per stage
  constexpr int PER_WAVE = GROUPS / NW;
  static_assert(GROUPS % NW == 0, "stage loads must split evenly over waves");
  static_assert(WM % 16 == 0 && WN % 16 == 0, "wavefront tile");
  static_assert(!DUAL || NT % 2 == 0, "SwiGLU tiles pair gate and up sub-tiles");
  constexpr int STAGE = ROWS * ROWB;           // bytes
  constexpr int NSW = NS + WD;                 // W ring depth
  constexpr int A_BYTES = A_ROWS * ROWB, W_BYTES = BN * ROWB;
  constexpr int GA = A_ROWS / RPI, GW = BN / RPI;
  constexpr int PWA = GA / NW, PWW = GW / NW;
  static_assert(!WD || (GA % NW == 0 && GW % NW == 0),
                "deep W ring: A and W loads must split evenly over waves");

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

  // Per-lane global source of load group g (rows g * RPI .. of the stage:
  // A rows first, then W rows).
  auto group_src = [&](int g) -> const uint16_t* {
    const int rr = lane / CPR, phys = lane % CPR;
    const int row = g * RPI + rr;  // row in the stage
    const int c = phys ^ lds_swz<KS>(row);
    if (row < A_ROWS) {
      const int r = row % BM;
      const int m = min(m0 + r, M - 1);  // rows past M load row M-1, never stored
      const uint16_t* base = (SPLIT && row >= BM) ? p.a_lo : p.a_hi;
      return base + (size_t)m * p.lda + c * 8;
    }
    const int r = row - A_ROWS;
    const int nn = min(DUAL ? n0 + (r % (BN / 2)) : n0 + r, N - 1);
    const uint16_t* base = (DUAL && r >= BN / 2) ? p.w2 : p.w;
    return base + (size_t)nn * K + c * 8;
  };
  const uint16_t* src[WD ? 1 : PER_WAVE];
  const uint16_t* srca[WD ? PWA : 1];
  const uint16_t* srcw[WD ? PWW : 1];
  if constexpr (WD) {
#pragma unroll
    for (int i = 0; i < PWA; i++) srca[i] = group_src(wave * PWA + i);
#pragma unroll
    for (int i = 0; i < PWW; i++) srcw[i] = group_src(GA + wave * PWW + i);
  } else {
#pragma unroll
    for (int i = 0; i < PER_WAVE; i++) src[i] = group_src(wave * PER_WAVE + i);
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
  auto issue_a = [&](int t) {
    unsigned char* st = smem + (t % NS) * A_BYTES;
    const int k0 = kbeg + t * KS;
#pragma unroll
    for (int i = 0; i < PWA; i++)
      __builtin_amdgcn_global_load_lds((const void*)(srca[i] + k0),
                                       (lds_ptr)(st + (wave * PWA + i) * 1024), 16, 0, 0);
  };
  auto issue_w = [&](int t) {
    unsigned char* st = smem + NS * A_BYTES + (t % NSW) * W_BYTES;
    const int k0 = kbeg + t * KS;
#pragma unroll
    for (int i = 0; i < PWW; i++)
      __builtin_amdgcn_global_load_lds((const void*)(srcw[i] + k0),
                                       (lds_ptr)(st + (wave * PWW + i) * 1024), 16, 0, 0);
  };
  auto frag = [&](const unsigned char* base, int r, int j = 0) -> bf16x8 {
    const int c = 4 * j + lane / 16;  // logical chunk of MFMA k-step j
    return *(const bf16x8*)(base + r * ROWB + ((c ^ lds_swz<KS>(r)) << 4));
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

  const int fr = lane % 16;
  // One K step: fragments from A stage sa and W stage sw, MFMAs.
  auto mma_step = [&](const unsigned char* sa, const unsigned char* sw) {
#pragma unroll
    for (int ks = 0; ks < KSUB; ks++) {
      bf16x8 bfrag[NT];
#pragma unroll
      for (int j = 0; j < NT; j++) bfrag[j] = frag(sw, b_tile_row(j) + fr, ks);
#pragma unroll
      for (int i = 0; i < MT; i++) {
        const int r = wm * WM + i * 16 + fr;
        const bf16x8 ahi = frag(sa, r, ks);
#pragma unroll
        for (int j = 0; j < NT; j++)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ahi, bfrag[j], acc[i][j], 0, 0, 0);
        if (SPLIT) {
          const bf16x8 alo = frag(sa + BM * ROWB, r, ks);
#pragma unroll
          for (int j = 0; j < NT; j++)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(alo, bfrag[j], acc[i][j], 0, 0, 0);
        }
      }
    }
  };
  if constexpr (WD) {
    // Issue order W0 A0 W1 A1 .. W(NS-2) A(NS-2) W(NS-1), then per step kt
    // A(kt+NS-1) W(kt+NS). Loads complete in issue order, so at step kt the
    // ones issued after A(kt) may stay in flight: W(kt+1 .. kt+NS-1) and
    // A(kt+1 .. kt+NS-2). Slots rewritten at step kt were last read at step
    // kt-1, which every wave has finished at the barrier.
#pragma unroll
    for (int t = 0; t < NS - 1; t++)
      if (t < nk) {
        issue_w(t);
        issue_a(t);
      }
    if (NS - 1 < nk) issue_w(NS - 1);
    for (int kt = 0; kt < nk; kt++) {
      const int aw = max(0, min(kt + NS - 1, nk - 1) - kt), aa = max(0, min(kt + NS - 2, nk - 1) - kt);
      wait_vmcnt(aw * PWW + aa * PWA);
      __builtin_amdgcn_s_barrier();
      if (kt + NS - 1 < nk) issue_a(kt + NS - 1);
      if (kt + NS < nk) issue_w(kt + NS);
      mma_step(smem + (kt % NS) * A_BYTES, smem + NS * A_BYTES + (kt % NSW) * W_BYTES);
    }
  } else {
#pragma unroll
  for (int t = 0; t < NS - 1; t++)
    if (t < nk) issue(t);
  for (int kt = 0; kt < nk; kt++) {
    const int ahead = min(NS - 2, nk - 1 - kt);  // stages still allowed in flight
    wait_vmcnt(ahead * PER_WAVE);
    __builtin_amdgcn_s_barrier();
    if (kt + NS - 1 < nk) issue(kt + NS - 1);
    const unsigned char* st = smem + (kt % NS) * STAGE;
    mma_step(st, st + A_ROWS * ROWB);
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
            const size_t at = ((size_t)head * p.ctx + P + m) * p.head_dim + h;
            if (!p.kv_bf16) cache[at] = v;
            else if (kv < p.kv_dim) p.kstage[(size_t)m * p.kv_dim + kv] = v;  // rounded after RoPE
            else ((uint16_t*)cache)[at] = f32_to_bf16_any(v);
          }
        }
      }
    }
  }
}

// ------------------------------------------------- pipelined form --
// Same operands, epilogues, tile order and split-K as gemm_kernel; the
// main loop is rebuilt around v_mfma_f32_32x32x16_bf16 for the large
// prefill shapes (measured faster there than the 16x16x32 tiles):
// * stages of KS (32 or 64) K values, rows of 2 KS bytes in LDS, filled by
//   the global-to-LDS DMA into NS buffers, one barrier per stage (the
//   dispatched shape: 256 x 256, 32-deep, 3 stages = 144 KiB, eight
//   wavefronts of 64 x 128);
// * a stage is KS / 16 sub-steps; the fragments of sub-step u + 1 are read
//   from LDS (double-buffered registers) between the MFMAs of sub-step u,
//   and a stage's refill DMA between those of its last sub-step;
// * at the last sub-step of stage t every wavefront has its reads of stage
//   t back, so after the barrier the DMA of stage t + NS reuses stage t's
//   buffer: NS - 1 stages in flight.
// Fragments (32x32x16): lane l reads row l % 32, 16-byte chunk
// 2 s + l / 32 of its stage row (s = sub-step). Chunk c of row r is stored
// at chunk c ^ swz(r): within each 16-lane LDS phase of a 128-bit read
// (lane quads of one bit parity per half wavefront), the rows that share
// banks land on distinct chunks (no bank conflicts counted on the GPU).
// Output of a 32x32 tile: lane l, element e holds
// C[8 (e / 4) + 4 (l / 32) + e % 4][l % 32].
template <int KS>
__device__ __forceinline__ int swz3(int r) {
  return KS == 32 ? (r >> 2) & 3 : (r >> 1) & 7;
}

template <int BM, int BN, int NS, int EPI, int PREC, int NW, int KS, int OCC>
__global__ __launch_bounds__(NW * WAVE, OCC) void gemm3_kernel(GemmParams p) {
  constexpr bool SPLIT = PREC == GEMM_SPLIT2;
  constexpr bool DUAL = EPI == GEMM_SWIGLU;
  constexpr int ROWB = 2 * KS, CPR = ROWB / 16, RPI = 1024 / ROWB;  // row bytes, chunks, rows per KiB
  constexpr int SUB = KS / 16;                 // MFMA sub-steps per stage
  constexpr int WGM = NW / 2;                  // wavefront rows x 2 columns
  constexpr int WM = BM / WGM, WN = BN / 2;
  constexpr int MT = WM / 32, NT = WN / 32;    // 32x32 tiles per wavefront
  constexpr int A_ROWS = BM * (SPLIT ? 2 : 1);
  constexpr int ROWS = A_ROWS + BN;
  constexpr int STAGE = ROWS * ROWB;
  constexpr int GROUPS = ROWS / RPI;           // 1 KiB DMA instructions per stage
  constexpr int PER_WAVE = GROUPS / NW;
  constexpr int NMFMA = MT * NT * (SPLIT ? 2 : 1);  // per sub-step
  constexpr int NREAD = MT * (SPLIT ? 2 : 1) + NT;  // fragment reads per sub-step
  static_assert(KS == 32 || KS == 64, "stage depth");
  static_assert(GROUPS % NW == 0 && WM % 32 == 0 && WN % 32 == 0, "tile shape");
  static_assert(!DUAL || NT % 2 == 0, "SwiGLU pairs gate and up tiles");
  static_assert(NMFMA > NREAD, "interleave needs an MFMA per fragment read, and one for the refill");

  extern __shared__ __attribute__((aligned(1024))) unsigned char smem[];
  // the wavefront index is uniform: in an SGPR, the DMA's LDS addresses are
  // scalar arithmetic (no readfirstlane per load)
  const int tid = threadIdx.x, lane = tid % WAVE, wave = __builtin_amdgcn_readfirstlane(tid / WAVE);
  const int wm = wave / 2, wn = wave % 2;
  const int cols = DUAL ? BN / 2 : BN;
  const int mtiles = (p.M + BM - 1) / BM, ntiles = (p.N + cols - 1) / cols;
  int m_tile, n_tile;
  tile_of(mtiles, ntiles, m_tile, n_tile, p.order);
  const int m0 = m_tile * BM, n0 = n_tile * cols;
  const int M = p.M, N = p.N, K = p.K;
  const int ksplit = gridDim.z, kper = ((K + KS - 1) / KS + ksplit - 1) / ksplit * KS;
  const int kbeg = blockIdx.z * kper, kend = min(K, kbeg + kper);
  const int nk = kend > kbeg ? (kend - kbeg) / KS : 0;
  if (nk == 0) {  // an empty K range of a split-K launch: its partial sums are zero
    if (EPI == GEMM_PARTIAL)
      for (int x = tid; x < BM * cols; x += NW * WAVE) {
        const int m = m0 + x / cols, n = n0 + x % cols;
        if (m < M && n < N) p.c[((size_t)blockIdx.z * M + m) * p.ldc + n] = 0.0f;
      }
    return;
  }

  // DMA sources of this lane for its PER_WAVE load groups
  const uint16_t* src[PER_WAVE];
#pragma unroll
  for (int i = 0; i < PER_WAVE; i++) {
    const int g = wave * PER_WAVE + i;
    const int row = g * RPI + lane / CPR;
    const int c = (lane % CPR) ^ swz3<KS>(row);
    if (row < A_ROWS) {
      const int m = min(m0 + row % BM, M - 1);  // rows past M load row M-1, never stored
      const uint16_t* base = (SPLIT && row >= BM) ? p.a_lo : p.a_hi;
      src[i] = base + (size_t)m * p.lda + c * 8;
    } else {
      const int r = row - A_ROWS;
      const int nn = min(DUAL ? n0 + (r % (BN / 2)) : n0 + r, N - 1);
      const uint16_t* base = (DUAL && r >= BN / 2) ? p.w2 : p.w;
      src[i] = base + (size_t)nn * K + c * 8;
    }
  }
  // DMA of stage t into buffer t % NS. Stages past the K range are issued
  // all the same (re-reading the first stage, into a buffer no later read
  // uses), so that every wait counts a constant number of newer loads.
  auto issue = [&](int t) {
    unsigned char* st = smem + (t % NS) * STAGE;
    const int k0 = kbeg + (t < nk ? t : 0) * KS;
#pragma unroll
    for (int i = 0; i < PER_WAVE; i++)
      __builtin_amdgcn_global_load_lds((const void*)(src[i] + k0),
                                       (lds_ptr)(st + (wave * PER_WAVE + i) * 1024), 16, 0, 0);
  };
  // fragment rows of this wavefront
  const int fr = lane % 32, fh = lane / 32;
  auto b_row = [&](int j) -> int {
    if (!DUAL) return wn * WN + j * 32;
    return (j < NT / 2 ? 0 : BN / 2) + wn * (WN / 2) + (j % (NT / 2)) * 32;
  };
  struct Frags {
    bf16x8 a[MT], al[SPLIT ? MT : 1], b[NT];
  };
  auto rd = [&](const unsigned char* st, int r, int sub) -> bf16x8 {
    const int c = 2 * sub + fh;
    return *(const bf16x8*)(st + r * ROWB + ((c ^ swz3<KS>(r)) << 4));
  };
  auto read_frags = [&](int u, Frags& F) {  // sub-step u = SUB t + sub
    const unsigned char* st = smem + ((u / SUB) % NS) * STAGE;
    const int sub = u % SUB;
#pragma unroll
    for (int i = 0; i < MT; i++) {
      const int r = wm * WM + i * 32 + fr;
      F.a[i] = rd(st, r, sub);
      if (SPLIT) F.al[i] = rd(st, BM + r, sub);
    }
#pragma unroll
    for (int j = 0; j < NT; j++) F.b[j] = rd(st, A_ROWS + b_row(j) + fr, sub);
  };

  f32x16 acc[MT][NT];
#pragma unroll
  for (int i = 0; i < MT; i++)
#pragma unroll
    for (int j = 0; j < NT; j++)
#pragma unroll
      for (int e = 0; e < 16; e++) acc[i][j][e] = 0.0f;

  // hi products of every tile, then the lo products: MT x NT independent
  // MFMAs separate the two that update one accumulator
  auto mfmas = [&](const Frags& F) {
#pragma unroll
    for (int i = 0; i < MT; i++)
#pragma unroll
      for (int j = 0; j < NT; j++)
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(F.a[i], F.b[j], acc[i][j], 0, 0, 0);
    if (SPLIT) {
#pragma unroll
      for (int i = 0; i < MT; i++)
#pragma unroll
        for (int j = 0; j < NT; j++)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(F.al[i], F.b[j], acc[i][j], 0, 0, 0);
    }
  };

  // prologue: stages 0 .. NS-1 in flight, stage 0 landed, its first fragments
  Frags F0, F1;
#pragma unroll
  for (int t = 0; t < NS; t++) issue(t);
  wait_vmcnt((NS - 1) * PER_WAVE);
  __builtin_amdgcn_s_barrier();
  read_frags(0, F0);
  // A sub-step within a stage: the MFMAs of u from `cur`, the fragments of
  // u + 1 (same stage) into `nxt`, one read per MFMA.
  // The fragment reads go out with the first MFMAs of a sub-step, so that
  // the rest of its MFMAs cover their latency; sched_barrier keeps every
  // MFMA of a sub-step on its side of the stage barrier.
  auto inner_step = [&](int u, Frags& cur, Frags& nxt) {
    read_frags(u + 1, nxt);
    mfmas(cur);
#pragma unroll
    for (int i = 0; i < NREAD; i++) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
    }
    __builtin_amdgcn_sched_group_barrier(0x008, NMFMA - NREAD, 0);
    __builtin_amdgcn_sched_barrier(0);
  };
  // The last sub-step of stage t: stage t + 1 landed (t + 2 .. may stay in
  // flight), every wavefront has its reads of stage t back: refill stage t's
  // buffer. The fragments of stage t + 1 go out first (the next sub-step
  // waits for them), the refill DMA after them, PER_MFMA per MFMA.
  auto last_step = [&](int u, Frags& cur, Frags& nxt) {
    const int t = u / SUB;
    wait_vmcnt((NS - 2) * PER_WAVE);
    __builtin_amdgcn_s_waitcnt(0xF | (7 << 4) | (0 << 8) | (3 << 14));  // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
    read_frags(u + 1, nxt);
    issue(t + NS);
    mfmas(cur);
#pragma unroll
    for (int i = 0; i < NREAD; i++) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
    }
    constexpr int DMA_MFMAS = NMFMA - NREAD;  // MFMAs that carry the refill
    constexpr int PER = (PER_WAVE + DMA_MFMAS - 1) / DMA_MFMAS;
#pragma unroll
    for (int i = 0; i < (PER_WAVE + PER - 1) / PER; i++) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);    // MFMA
      __builtin_amdgcn_sched_group_barrier(0x020, PER, 0);  // DMA
    }
    __builtin_amdgcn_sched_group_barrier(0x008, DMA_MFMAS - (PER_WAVE + PER - 1) / PER, 0);
    __builtin_amdgcn_sched_barrier(0);
  };
  // every stage but the last: SUB sub-steps (fragment registers alternate,
  // SUB is even), the last one refills
  for (int t = 0; t + 1 < nk; t++) {
#pragma unroll
    for (int s = 0; s < SUB; s += 2) {
      inner_step(SUB * t + s, F0, F1);
      if (s + 2 < SUB) inner_step(SUB * t + s + 1, F1, F0);
      else last_step(SUB * t + s + 1, F1, F0);
    }
  }
  {  // the last stage: no refill, and its final sub-step reads nothing
    const int u = SUB * (nk - 1);
#pragma unroll
    for (int s = 0; s + 2 < SUB; s += 2) {
      inner_step(u + s, F0, F1);
      inner_step(u + s + 1, F1, F0);
    }
    inner_step(u + SUB - 2, F0, F1);
    mfmas(F1);
  }
  __builtin_amdgcn_s_waitcnt(0);  // no DMA left in flight into this block's LDS

  // Epilogue
  const int P = (EPI == GEMM_QKV) ? *p.pos : 0;
  const int ecol = lane % 32, erow = (lane / 32) * 4;
  const bool out_split = p.c_lo != nullptr;
#pragma unroll
  for (int i = 0; i < MT; i++) {
#pragma unroll
    for (int j = 0; j < (DUAL ? NT / 2 : NT); j++) {
      const int n = DUAL ? n0 + wn * (WN / 2) + j * 32 + ecol : n0 + wn * WN + j * 32 + ecol;
      if (n >= N) continue;
#pragma unroll
      for (int e = 0; e < 16; e++) {
        const int m = m0 + wm * WM + i * 32 + 8 * (e / 4) + erow + (e % 4);
        if (m >= M) continue;
        const float v = acc[i][j][e];
        if (EPI == GEMM_STORE) {
          p.c[(size_t)m * p.ldc + n] = v;
        } else if (EPI == GEMM_RESIDUAL) {
          p.c[(size_t)m * p.ldc + n] += v;
        } else if (EPI == GEMM_PARTIAL) {
          p.c[((size_t)blockIdx.z * M + m) * p.ldc + n] = v;
        } else if (EPI == GEMM_SWIGLU) {
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
            const size_t at = ((size_t)head * p.ctx + P + m) * p.head_dim + h;
            if (!p.kv_bf16) cache[at] = v;
            else if (kv < p.kv_dim) p.kstage[(size_t)m * p.kv_dim + kv] = v;  // rounded after RoPE
            else ((uint16_t*)cache)[at] = f32_to_bf16_any(v);
          }
        }
      }
    }
  }
}

template <int BM, int BN, int NS, int EPI, int PREC, int NW, int KS, int OCC = 1>
void launch3(const GemmParams& p0, int splits, hipStream_t s) {
  static const int order = getenv("STRASGPT_GEMM_ORDER") ? atoi(getenv("STRASGPT_GEMM_ORDER")) : 3;
  GemmParams p = p0;
  p.order = order;
  const int cols = EPI == GEMM_SWIGLU ? BN / 2 : BN;
  const int tiles = ((p.N + cols - 1) / cols) * ((p.M + BM - 1) / BM);
  constexpr size_t shm = (size_t)NS * (BM * (PREC == GEMM_SPLIT2 ? 2 : 1) + BN) * 2 * KS;
  static_assert(shm <= 160 * 1024, "GEMM stages exceed LDS");
  static bool attr = false;
  if (!attr) {
    HIP_CHECK(hipFuncSetAttribute((const void*)gemm3_kernel<BM, BN, NS, EPI, PREC, NW, KS, OCC>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm));
    attr = true;
  }
  hipLaunchKernelGGL((gemm3_kernel<BM, BN, NS, EPI, PREC, NW, KS, OCC>), dim3(tiles, 1, splits),
                     dim3(NW * WAVE), shm, s, p);
}

template <int BM, int BN, int NS, int EPI, int PREC, int OCC = 0, int KS = 32, int WD = 0, int NW = 4>
void launch(const GemmParams& p, int splits, hipStream_t s) {
  const int cols = EPI == GEMM_SWIGLU ? BN / 2 : BN;
  const int tiles = ((p.N + cols - 1) / cols) * ((p.M + BM - 1) / BM);
  constexpr int rows = BM * (PREC == GEMM_SPLIT2 ? 2 : 1) + BN;
  constexpr size_t shm = ((size_t)NS * rows + (size_t)WD * BN) * KS * 2;
  static_assert(shm <= 160 * 1024, "GEMM stages exceed LDS");
  static bool attr = false;
  if (!attr) {
    HIP_CHECK(hipFuncSetAttribute((const void*)gemm_kernel<BM, BN, NS, EPI, PREC, OCC, KS, WD, NW>,
                                  hipFuncAttributeMaxDynamicSharedMemorySize, (int)shm));
    attr = true;
  }
  hipLaunchKernelGGL((gemm_kernel<BM, BN, NS, EPI, PREC, OCC, KS, WD, NW>), dim3(tiles, 1, splits),
                     dim3(NW * WAVE), shm, s, p);
}

// Tile shape forced by STRASGPT_GEMM_TILE ("256x256", "128x256", "128x128",
// "64x128x64", "64x128x64s4", "64x128", "64x64", "64x64x64s6"), for tests that run every
// shape on small models; 0 = by size.
int forced_tile() {
  const char* v = getenv("STRASGPT_GEMM_TILE");
  if (!v || !*v) return 0;
  if (!strcmp(v, "256x256")) return 7;
  if (!strcmp(v, "128x256")) return 4;
  if (!strcmp(v, "128x128")) return 3;
  if (!strcmp(v, "64x128x64")) return 5;
  if (!strcmp(v, "64x128x64s4")) return 6;
  if (!strcmp(v, "64x128")) return 2;
  if (!strcmp(v, "64x64")) return 1;
  if (!strcmp(v, "64x64x64s6")) return 8;
  if (!strcmp(v, "128x384")) return 9;
  ST_DIE("STRASGPT_GEMM_TILE must be 256x256, 128x384, 128x256, 128x128, 64x128x64, 64x128x64s4, 64x128, "
         "64x64 or 64x64x64s6");
}

template <int EPI, int PREC>
void dispatch_tile(const GemmParams& p, int splits, hipStream_t s) {
  // Measured on MI355X, bf16x2, with the weights coming from HBM (caches
  // evicted before each launch, as in a prefill pass):
  // * from 192 tiles of 256 x 256 (3/4 of the CUs; M >= 2048 on the
  //   d = 5120 projections, M >= 512 on the wide FFN ones), the 32x32x16
  //   kernel with eight wavefronts (two per SIMD) is 5-25% faster than the
  //   16x16x32 tiles (Mistral-Small-24B shapes at M = 2048: gate/up 23.4%
  //   of the bf16 peak in algorithmic flops, QKV 21.2%); with fewer tiles,
  //   or a last round of blocks that leaves more than a quarter of the CUs
  //   idle (320 blocks = 1.25 rounds), part of the chip idles and it loses;
  //   the gate/up SwiGLU GEMM is the exception from 128 tiles (half the CUs
  //   in one round): Qwen3-4B shape at M = 512 (152 tiles), 110 us against
  //   118 for the best 16x16x32 tiles; QKV, O and down at 20-48 tiles lose
  //   by 1.3-2.1x;
  // * from about 4 blocks of 128 x 256 per CU, 128 x 256 with 32-deep
  //   stages and two blocks per CU (fewest stage bytes per MFMA);
  // * below that, 64 x 128 tiles with 64-deep stages: 128-byte row segments
  //   per DMA lane group move ~1.8x the bytes per cycle of 64-byte ones.
  //   With more than one block per CU: two blocks per CU, a 2-stage A ring
  //   and a 3-stage W ring (80 KiB; the blocks sharing a W tile request it
  //   together, so W needs the longer cover); with at most one block per
  //   CU: one block with a 4-stage ring. 1.2-2.3x over the 32-deep shapes
  //   on the M = 256 and 512 projections;
  // * K not a multiple of 64 and tiny grids keep the 32-deep shapes.
  const int cols = EPI == GEMM_SWIGLU ? 64 : 128;
  const long big = (long)((p.N + cols - 1) / cols) * ((p.M + 127) / 128) * splits;
  const long wide = (long)((p.N + 2 * cols - 1) / (2 * cols)) * ((p.M + 127) / 128) * splits;
  const long small = (long)((p.N + cols - 1) / cols) * ((p.M + 63) / 64) * splits;
  const long huge = (long)((p.N + 2 * cols - 1) / (2 * cols)) * ((p.M + 255) / 256) * splits;
  int shape = forced_tile();
  if ((shape == 5 || shape == 6 || shape == 8) && p.K % 64) shape = 2;
  if (!shape) {
    const long rounds = (huge + 255) / 256;  // rounds of one 256 x 256 block per CU
    // a few rows (short prompts): the weights are the whole cost; 64-wide
    // tiles with a 6-stage ring of 64-deep steps keep the most weight bytes
    // in flight (SwiGLU at 8 rows, Llama-3.2-1B shape: 23.0 us against 25.0
    // for 64 x 128 tiles)
    if (EPI == GEMM_SWIGLU && p.M <= kSmallM && p.K % 64 == 0) shape = 8;
    else if ((huge >= 192 && 4 * huge >= 3 * 256 * rounds) || (EPI == GEMM_SWIGLU && huge >= 128 && huge <= 256)) {
      shape = 7;
      // 128 x 384 tiles where their last round of blocks is at least a
      // tenth fuller (bf16x2): the Mistral-Small-24B QKV projection at
      // M = 2048 (N = 6144) is 256 of them against 192 of 256 x 256, 240
      // against 264 us stand-alone with the weights from HBM; the Qwen3-4B
      // gate/up SwiGLU GEMM at M = 512, 204 against 152 tiles, 115 against
      // 127 us
      const long t384 = (long)((p.N + 3 * cols - 1) / (3 * cols)) * ((p.M + 127) / 128) * splits;
      const long r384 = (t384 + 255) / 256;
      if (PREC == GEMM_SPLIT2 && 10 * t384 * rounds >= 11 * huge * r384) shape = 9;
    }
    else if (wide >= 1024) shape = 4;
    else if (p.K % 64 == 0 && small > 256) shape = 5;
    else if (p.K % 64 == 0 && small >= 64) shape = 6;
    else shape = big >= 512 ? 3 : big >= 192 ? 2 : 1;
  }
  switch (shape) {
    case 7: launch3<256, 256, 3, EPI, PREC, 8, 32, 2>(p, splits, s); break;
    case 9:  // 128 x 384, eight wavefronts of 32 x 192 (bf16x2: with single
      // bf16 operands a sub-step has more fragment reads than MFMAs)
      if constexpr (PREC == GEMM_SPLIT2) launch3<128, 384, 3, EPI, PREC, 8, 32, 1>(p, splits, s);
      else launch3<256, 256, 3, EPI, PREC, 8, 32, 2>(p, splits, s);
      break;
    case 4: launch<128, 256, 2, EPI, PREC, 2>(p, splits, s); break;
    case 5: launch<64, 128, 2, EPI, PREC, 2, 64, 1>(p, splits, s); break;
    case 6: launch<64, 128, 4, EPI, PREC, 1, 64>(p, splits, s); break;
    case 8: launch<64, 64, 6, EPI, PREC, 1, 64>(p, splits, s); break;
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

// Split count that puts the 64 x 128 tiles with 64-deep stages (two blocks
// per CU) in one round of at least 3/4 of the 512 block slots; 0 if none
// does. Each split adds a set of M x N partial sums to write and read back,
// and a second, partial round of blocks costs a whole K range more, so the
// largest count that still fits one round wins. Measured stand-alone with
// the weights from HBM, partial sums added by the next kernel: Qwen3-4B O
// and down projections at M = 512 (160 tiles), 3 splits 35.5 and 66.3 us
// against 42.2 and 74.8 with 4 (1.25 rounds); the MXFP4 MoE O projection at
// M = 256 (92 tiles), 5 splits 30.8 us against 36.7 with 6; its QKV
// projection (160 tiles), 3 splits and the split epilogue 29.2 us against
// 35.2 unsplit.
int round_splits(int M, int N, int K) {
  if (K % 64) return 0;
  const long t64 = (long)((N + 127) / 128) * ((M + 63) / 64);
  if (t64 >= 512) return 0;
  int s = (int)std::min<long>(8, 512 / t64);
  while (s > 1 && K / 64 < 4 * s) s--;  // at least 4 K steps per split
  return 4 * t64 * s >= 3 * 512 ? s : 0;
}

}  // namespace

int gemm_splits(int M, int N, int K) {
  // Reductions of K >= 4096 over many rows: the fewest splits that give
  // the 256 x 256 kernel whole rounds of blocks (at least 3/4 of the last
  // one used). Its tiles re-read the activations a quarter as often as
  // 64 x 128 ones: on the Mistral-Small-24B down projection (M = 2048,
  // K = 32768) the 64 x 128 tiles moved 12x the algorithmic HBM bytes; its
  // O projection (M = 2048, K = 4096, 160 tiles, 3 splits) takes 156 us
  // against 214 for the unsplit 64 x 128 tiles.
  if (K >= 4096) {
    const long t256 = (long)((N + 255) / 256) * ((M + 255) / 256);
    for (int s = 1; s <= 8 && K / (BK * s) >= 4; s++) {
      const long blocks = t256 * s, rounds = (blocks + 255) / 256;
      if (blocks >= 192 && 4 * blocks >= 3 * 256 * rounds) return s;
    }
  }
  if (const int s = round_splits(M, N, K)) return s;
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

namespace {

// Epilogue of a split-K QKV or SwiGLU GEMM (few rows): thread (m, n) sums
// the partials in split order and applies the fused GEMM epilogue (QKV:
// the q row, the key row (or its staging row for a bf16 cache) and the
// value row at position P + m; SwiGLU: silu(gate) * up stored as the next
// GEMM's hi/lo planes).
template <int EPI>
__global__ __launch_bounds__(256) void split_epilogue_kernel(GemmParams p, const float* part, const float* part2,
                                                             int splits) {
  const int M = p.M, N = EPI == GEMM_SWIGLU ? p.N : p.q_dim + 2 * p.kv_dim;
  const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (size_t)M * N) return;
  const int m = (int)(idx / N), n = (int)(idx % N);
  // the partials of four splits requested before their sums (in split order)
  auto sum_splits = [&](const float* pp) {
    float acc = 0.0f;
    for (int sp = 0; sp < splits; sp += 4) {
      float x[4];
#pragma unroll
      for (int u = 0; u < 4; u++) x[u] = pp[((size_t)min(sp + u, splits - 1) * M + m) * N + n];
#pragma unroll
      for (int u = 0; u < 4; u++)
        if (sp + u < splits) acc += x[u];
    }
    return acc;
  };
  const float v = sum_splits(part);
  if (EPI == GEMM_SWIGLU) {
    const float u = sum_splits(part2);
    store_split(p.c_hi, p.c_lo, (size_t)m * p.ldc + n, silu_mul(v, u), p.c_lo != nullptr);
  } else if (n < p.q_dim) {
    p.q[(size_t)m * p.q_dim + n] = v;
  } else {
    const int P = *p.pos;
    const int kv = n - p.q_dim;
    float* cache = kv < p.kv_dim ? p.kcache : p.vcache;
    const int j2 = kv < p.kv_dim ? kv : kv - p.kv_dim;
    const int head = j2 / p.head_dim, h = j2 % p.head_dim;
    const size_t at = ((size_t)head * p.ctx + P + m) * p.head_dim + h;
    if (!p.kv_bf16) cache[at] = v;
    else if (kv < p.kv_dim) p.kstage[(size_t)m * p.kv_dim + kv] = v;  // rounded after RoPE
    else ((uint16_t*)cache)[at] = f32_to_bf16_any(v);
  }
}

}  // namespace

int gemm_small_splits(int M, int N, int K, int epi, size_t ws_floats) {
  if (M > kSmallM && epi == GEMM_QKV) {  // mid-size prompts: one full round of split tiles
    int sp = std::max(1, round_splits(M, N, K));
    while (sp > 1 && (size_t)sp * M * N > ws_floats) sp--;
    return sp;
  }
  if (M > kSmallM || (epi != GEMM_QKV && epi != GEMM_SWIGLU) || K % 64) return 1;
  const int tiles = (N + 127) / 128 * (epi == GEMM_SWIGLU ? 2 : 1);  // 64 x 128 tiles of the partial GEMMs
  int sp = std::min(8, std::max(1, (256 + tiles - 1) / tiles));
  while (sp > 1 && K / 64 < 4 * sp) sp--;  // at least 4 K steps per split
  while (sp > 1 && (size_t)sp * M * N * (epi == GEMM_SWIGLU ? 2 : 1) > ws_floats) sp--;
  return sp;
}

void gemm_small(const GemmParams& p, int epi, int prec, int splits, float* ws, hipStream_t s) {
  if (splits < 2 || (epi != GEMM_QKV && epi != GEMM_SWIGLU)) ST_DIE("gemm_small: split QKV or SwiGLU only");
  const int N = epi == GEMM_SWIGLU ? p.N : p.q_dim + 2 * p.kv_dim;
  if (epi == GEMM_QKV && p.N != N) ST_DIE("GEMM QKV column count mismatch");
  GemmParams q = p;
  q.w2 = nullptr;
  q.c = ws;
  q.ldc = N;
  gemm(q, GEMM_PARTIAL, prec, splits, s);
  float* ws2 = ws + (size_t)splits * p.M * N;
  if (epi == GEMM_SWIGLU) {
    q.w = p.w2;
    q.c = ws2;
    gemm(q, GEMM_PARTIAL, prec, splits, s);
  }
  const size_t threads = (size_t)p.M * N;
  const dim3 grid((unsigned)((threads + 255) / 256));
  if (epi == GEMM_SWIGLU)
    hipLaunchKernelGGL(split_epilogue_kernel<GEMM_SWIGLU>, grid, dim3(256), 0, s, p, ws, ws2, splits);
  else
    hipLaunchKernelGGL(split_epilogue_kernel<GEMM_QKV>, grid, dim3(256), 0, s, p, ws, nullptr, splits);
  HIP_CHECK(hipGetLastError());
}

void gemm(const GemmParams& p, int epi, int prec, int splits, hipStream_t s) {
  check(p, epi, prec, splits);
  if (prec == GEMM_SPLIT2) dispatch<GEMM_SPLIT2>(p, epi, splits, s);
  else if (prec == GEMM_BF16) dispatch<GEMM_BF16>(p, epi, splits, s);
  else ST_DIE("unknown GEMM precision");
  HIP_CHECK(hipGetLastError());
}

}  // namespace sg
