// Host-side launch interface of the gfx950 kernels. Every launcher checks
// on the host that the shapes fit what its kernel assumes (alignment,
// multiples, shared-memory limits) and dies with a message otherwise, so
// no kernel is launched on operands it would index out of bounds.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace sg {

// ---------------------------------------------------------------- GEMV --
// One activation row (decode step) against a bf16 [N][K] weight matrix,
// fp32 accumulation. Optional RMSNorm of the input row (the reference's
// rmsnorm, source/transformer.c:978-999) is computed by every block.
enum GemvEpilogue {
  GEMV_STORE = 0,    // y[n] = acc
  GEMV_RESIDUAL = 1, // y[n] += acc                 (O-proj, down-proj)
  GEMV_QKV = 2,      // rows -> q | raw k | v-cache (fused QKV projection)
  GEMV_SWIGLU = 3,   // y[n] = silu(gate_n . x) * (up_n . x)
};

struct GemvParams {
  const uint16_t* w;      // [N][K] bf16
  const uint16_t* w2;     // up matrix for GEMV_SWIGLU, else null
  const float* x;         // [K]
  const uint16_t* norm_w; // RMSNorm weight [K] or null (no norm)
  float eps;
  int N, K;
  float* y;
  // GEMV_QKV destinations
  float* q;        // [q_dim]
  float* kraw;     // [kv_dim]  (pre-norm, pre-RoPE keys of this step)
  float* vcache;   // this layer's [kv_heads][ctx][head_dim] (bf16 when kv_bf16)
  const int* pos;  // device: cache position of this step
  int q_dim, kv_dim, head_dim, ctx;
  int kv_bf16;     // the cache stores bf16 (round to nearest even)
  // Split-K scratch for rows longer than one LDS stage (residual epilogue):
  // partial sums [ranges][N] and one arrival counter per block, zero
  // between launches (kGemvCounters of them). Without it such rows take the
  // chunked form.
  float* part;
  unsigned* counters;
  // Multi-row form (gemv_rows): M activation rows x[m][K] (row stride K),
  // outputs y[m][N] (row stride N), q[m][q_dim]; QKV keys of row m go to
  // kcache at position *pos + m (fp32 cache) or to kstage[m][kv_dim] (bf16
  // cache: rounded after their RoPE), values to vcache at *pos + m.
  int M;
  float* kcache;
  float* kstage;
};
constexpr int kGemvCounters = 4096;
void gemv(const GemvParams& p, int epilogue, hipStream_t s);
// Prompts of at most kRowsMax tokens: every weight row streamed once into
// fp32 FMAs for all M rows (the decode GEMV's arithmetic per row), with the
// RMSNorm of each input row fused in (p.norm_w); rows longer than one LDS
// stage split over K (residual epilogue, p.part with kRowsMax * N floats
// per range, p.counters). False when the shape is not supported (the
// caller then runs the prefill GEMMs).
constexpr int kRowsMax = 8;
bool gemv_rows(const GemvParams& p, int epilogue, hipStream_t s);
// Whether gemv_rows takes M rows of length K (norm: with the RMSNorm; rows
// without it may split over K when the residual scratch is given).
bool gemv_rows_fit(int M, int K, bool norm);

// MXFP4 expert GEMV rows (decode MoE). Rows of expert e are
// [N][K/32][16] code bytes and [N][K/32] E8M0 exponents.
struct MoeGemvParams {
  const uint8_t* blocks;   // [E][N][K/2]
  const uint8_t* scales;   // [E][N][K/32]
  const uint8_t* blocks2;  // up (SWIGLU) or null
  const uint8_t* scales2;
  const float* x;          // SWIGLU: [tokens][K]; DOWN: [tokens][topk][K]
  const int* expert;       // [tokens][topk] selected expert ids
  const float* weight;     // [tokens][topk] routing weights (down-proj only)
  int tokens, topk, N, K;
  float* y;                // SWIGLU: [tokens*topk][N]; DOWN: y[t][n] += routed sum
  // Decode (one token, E <= 64): router logits [E] instead of expert /
  // weight; each block selects the top-k itself.
  const float* logits;
  int E;
};
// Decode router: logits[e] = W_r[e] . RMSNorm(x) for one token, and the
// normalised row into xn (read by the expert kernels). E <= 64, d <= 8192.
void moe_route_logits(const float* x, const uint16_t* norm_w, float eps, const uint16_t* router, int E, int d,
                      float* logits, float* xn, hipStream_t s);
bool moe_route_logits_supported(int E, int topk, int d);
void moe_gemv_swiglu(const MoeGemvParams& p, hipStream_t s);
void moe_gemv_down(const MoeGemvParams& p, hipStream_t s);
// Prefill MoE: slots grouped by expert, then grouped MXFP4 GEMMs.
// order[offs[e] .. offs[e+1]) lists the slots routed to expert e in
// increasing order (offs has E + 1 entries).
void moe_group(const int* sel, int n, int E, int* offs, int* order, hipStream_t s);
struct MoeGemmParams {
  const uint8_t *blocks, *scales;    // [E][N][K/32] x 16 bytes, [E][N][K/32]
  const uint8_t *blocks2, *scales2;  // second matrix of a SwiGLU pair, or null
  const float* a;                    // rows: a[token] (a_per_token) or a[slot], K floats
  int a_per_token;
  const int *offs, *order;           // moe_group output
  int slots, topk, E, N, K;
  float* y;                          // [slot][N]: silu(g) * u, or the product
  // optional: A as bf16 hi/lo planes; with them the pipelined kernel runs
  // (needs K % 64 == 0, N % 16 == 0). a_per_token: one row per token
  // ([T][K], row order[i] / topk read for expert-order row i); else the
  // rows in expert order ([slots][K], row i = the row of slot order[i]:
  // moe_gather_split, or y_hi/y_lo of the gate/up GEMM)
  uint16_t *a_hi, *a_lo;
  // optional, SwiGLU pair on the pipelined kernel: silu(g) * u written as
  // bf16 hi/lo planes in expert order ([slots][N], the next GEMM's A)
  // instead of y
  uint16_t *y_hi, *y_lo;
};
void moe_group_gemm(const MoeGemmParams& p, hipStream_t s);
// a_hi/a_lo[i] = split of the A row of slot order[i] (a[order[i] / topk] when
// a_per_token, else a[order[i]]), i < slots (for an A in expert order when
// the previous GEMM could not write its planes).
void moe_gather_split(const MoeGemmParams& p, hipStream_t s);
// Whether moe_group_gemm takes the pipelined kernel for p (a_hi/a_lo set,
// K % 64 == 0, K <= 8192, N % 16 == 0, 16-byte aligned operands).
bool moe_group_gemm2_ok(const MoeGemmParams& p);
// The device MXFP4 decode of the expert kernels on `nblocks` blocks of 32
// values (16 code bytes + 1 E8M0 scale each): out[32 b + i] (test hook);
// bf16_tiles: the grouped prefill GEMM's bf16 conversion, widened back.
void mxfp4_decode(const uint8_t* codes, const uint8_t* scales, int nblocks, float* out, int bf16_tiles,
                  hipStream_t s);

// ---------------------------------------------------------------- GEMM --
// C[M][N] = A[M][K] x W[N][K]^T (bf16 weights) on MFMA. A is given as two
// bf16 planes, hi = bf16(a) and lo = bf16(a - hi), written by the kernel
// that produced the activations; GEMM_SPLIT2 multiplies both planes,
// GEMM_BF16 only hi.
enum GemmPrecision { GEMM_SPLIT2 = 0, GEMM_BF16 = 1 };
enum GemmEpilogue {
  GEMM_STORE = 0,    // C[m][n] = acc
  GEMM_RESIDUAL = 1, // C[m][n] += acc
  GEMM_QKV = 2,      // q[m][n] | k-cache | v-cache rows at position P+m
  GEMM_SWIGLU = 3,   // (c_hi, c_lo)[m][n] = split(silu(A.Wg_n) * (A.Wu_n))
  GEMM_PARTIAL = 4,  // C[split][m][n] = partial sum of this K split
};
struct GemmParams {
  const uint16_t* a_hi;  // [M][lda] bf16
  const uint16_t* a_lo;  // [M][lda] bf16 (bf16x2 only)
  int lda;
  const uint16_t* w;   // [N][K]
  const uint16_t* w2;  // up matrix for GEMM_SWIGLU
  int M, N, K;
  float* c;            // [M][ldc] (PARTIAL: [splits][M][ldc])
  int ldc;
  uint16_t* c_hi;      // GEMM_SWIGLU output planes [M][ldc]
  uint16_t* c_lo;      //   (c_lo may be null: hi plane only)
  // GEMM_QKV
  float* q; float* kcache; float* vcache; const int* pos;
  int q_dim, kv_dim, head_dim, ctx;
  // bf16 cache (kv_bf16): values stored rounded into vcache (as bf16), raw
  // keys into kstage [M][kv_dim] fp32 (qk_norm_rope rounds them after RoPE)
  int kv_bf16;
  float* kstage;
  int order;           // tile order of the 256 x 256 kernel (set by the launcher)
};
void gemm(const GemmParams& p, int epilogue, int precision, int splits, hipStream_t s);
// Prompts of at most kSmallM rows: the QKV (or SwiGLU) GEMM as split-K
// partial GEMMs (64 x 128 tiles; enough blocks to keep weight bytes in
// flight on every CU) into ws, then one epilogue kernel that sums the
// partials in split order and applies the fused epilogue. The split count
// (1: use gemm) keeps at least 4 K steps per split and fits ws_floats.
// Llama-3.2-1B shape, 8 rows: QKV 22.4 -> 13.6 us (the fused GEMM has 48
// blocks of 64 x 64); the runtime keeps the fused SwiGLU GEMM, which was
// faster than its split form (23 vs 32 us). Above kSmallM rows the QKV GEMM
// splits when that fills one round of 64 x 128 tiles at two per CU (MXFP4
// MoE shape at 256 rows: 3 splits, 35.2 -> 29.2 us with the epilogue).
constexpr int kSmallM = 32;
int gemm_small_splits(int M, int N, int K, int epilogue, size_t ws_floats);
void gemm_small(const GemmParams& p, int epilogue, int precision, int splits, float* ws, hipStream_t s);
// Split-K factor that fills the CUs for an M x N output (1: no split).
int gemm_splits(int M, int N, int K);

// -------------------------------------------------------- elementwise --
void embed(const int* tok, int T, const uint16_t* table, int d, float* x, hipStream_t s);
void rmsnorm_rows(const float* x, const uint16_t* w, float* y, int rows, int d,
                  float eps, hipStream_t s);
// Row-wise: x += sum over s < splits of part[s] (in order; residual add of a
// split-K projection), then, if w is given, the reference RMSNorm of x
// written as fp32 (y, optional) and/or as bf16 hi/lo planes (y_hi, y_lo
// optional) for the next GEMM.
struct NormParams {
  float* x;
  const float* part;  // [splits][rows][d] or null
  int splits;
  // MoE routed sum or null: x[r] += sum over j in top-k order of
  // fmaf(routed_w[r topk + j], routed[r topk + j][.], .) (after the partials)
  const float* routed;
  const float* routed_w;
  int topk;
  const uint16_t* w;  // norm weight or null (residual only)
  float eps;
  int rows, d;
  float* y;
  uint16_t* y_hi;
  uint16_t* y_lo;
};
void residual_norm(const NormParams& p, hipStream_t s);
// Per-head RMSNorm (if norm weights given) and RoPE, in place, on T rows of
// q ([T][heads*hd]) and on the T new key rows of one layer's k-cache. With
// a bf16 cache (kstage given) the raw keys come from kstage [T][kv_heads*hd]
// and the results are stored rounded into the bf16 cache.
// The bf16 planes of the attention kernels' key/value operands: K [kv][ctx]
// [hd] hi/lo, V^T [kv][hd][ctx_pad] hi/lo, filled from the cache rows (the
// values from vcache: fp32, or bf16 with kv_bf16).
struct PlaneRows {
  uint16_t *khi, *klo, *vthi, *vtlo;
  const void* vcache;
  int ctx_pad, kv_bf16;
};

// With planes: also writes rows P .. P + T - 1 of the planes (the finished
// keys, the values) as attention_split_rows would; returns false where the
// head size takes the loop form, which writes no planes.
bool qk_norm_rope(float* q, int q_heads, float* kcache, int kv_heads, int T,
                  const int* pos, int ctx, int hd, const uint16_t* qn,
                  const uint16_t* kn, float eps, const float* rope,
                  int pair_bound, int pair_offset, int pair_stride, const float* kstage,
                  const PlaneRows* planes, hipStream_t s);

// ---------------------------------------------------------- attention --
struct AttnParams {
  const float* q;        // [T][q_heads*hd]
  const float* kcache;   // layer base [kv_heads][ctx][hd] (bf16 when kv_bf16)
  const float* vcache;
  int kv_bf16;
  float* out;            // decode: [q_heads*hd] fp32; prefill without out_hi: [T][q_heads*hd] fp32
  uint16_t* out_hi;      // prefill: [T][q_heads*hd] bf16 planes (O-GEMM input)
  uint16_t* out_lo;      //   (out_lo may be null)
  const int* pos;        // device: position of the first query (cached count)
  int T, q_heads, kv_heads, hd, ctx;
  int q0;                // prefill: the first query is at position *pos + q0
  // decode only: raw key of this step and QK-norm/RoPE inputs
  const float* kraw;     // [kv_heads*hd] or null
  float* kcache_w;       // k-cache (writable) for the processed key
  const uint16_t* qn;
  const uint16_t* kn;
  float eps;
  const float* rope;
  int pair_bound, pair_offset, pair_stride;
  // the layer's cache rows as bf16 planes (the split-bf16 prefill kernel's
  // and the decode kernel's operands), K [kv_heads][ctx][hd] (hi, lo) and
  // V transposed [kv_heads][hd][ctx_pad]; decode writes row P into them
  const uint16_t* khi;
  const uint16_t* klo;
  const uint16_t* vthi;
  const uint16_t* vtlo;
  int ctx_pad;           // ctx rounded up to a multiple of 32
  float* partial;        // [q_heads][splits][hd + 2]
  int splits;            // decode: blocks per kv head, at most (attention_decode_chunks)
  unsigned* counters;    // [kv_heads], zero between launches
};
void attention_prefill(const AttnParams& p, hipStream_t s);
// variant 0: split-bf16 matrix cores (16 or 32 queries per wavefront by the
// grid size), 1: fp32 matrix cores, 2 / 3: split bf16 with 16 / 32 queries
void attention_prefill_variant(const AttnParams& p, int variant, hipStream_t s);
// Cache rows [r0, r1) of every kv head of one layer into the bf16 planes the
// split-bf16 prefill kernel reads (AttnParams khi .. vtlo).
// With a bf16 cache (kv_bf16) the rows are bf16 already: hi = the row, lo = 0.
void attention_split_rows(const float* kcache, const float* vcache, uint16_t* khi, uint16_t* klo,
                          uint16_t* vthi, uint16_t* vtlo, int kv_heads, int ctx, int ctx_pad, int hd,
                          int r0, int r1, int kv_bf16, hipStream_t s);
void attention_decode(const AttnParams& p, hipStream_t s);
int attention_decode_chunks(int kv_heads);
// Sets the decode kernels' LDS limits; called once per device before use.
void attention_init();

// ------------------------------------------------------------- argmax --
// First index of the maximum (reference source/sampler.c:92-102): block
// partials, then one block writes out[0], appends to seq[*seq_len] (if seq)
// and bumps *pos_inc (if given) so that a replayed decode step advances.
struct ArgmaxParams {
  const float* x;
  int n;
  float* part_v;   // [blocks]
  int* part_i;     // [blocks]
  int* out;        // next token
  int* seq;        // token log or null
  int* seq_len;    // device counter or null
  int* pos_inc;    // device position to increment or null
};
void argmax(const ArgmaxParams& p, hipStream_t s);
int argmax_blocks();

// ----------------------------------------------------------- sampling --
// The reference's sampler_sample (source/sampler.c:234-337) on device
// logits: presence penalty, temperature 0 (argmax) or softmax, coin, top-k,
// top-p, renormalisation and the multinomial draw; writes the token like
// the argmax (out, seq, pos_inc).
struct SampleParams {
  const float* logits;
  int V;
  float temperature;
  int top_k;
  float top_p;
  float penalty;
  unsigned char* presence;       // [V] tokens seen (marked before the penalty)
  const int* prev;               // previous token on the device, or null:
  int prev_value;                //   then this one (< 0: none)
  unsigned long long* rng;       // xorshift64* state, advanced once per non-greedy draw
  // work buffers
  float* y;                      // [V]
  float* part;                   // [512]
  unsigned* keys;                // [V] x 2 and int [V] x 2: the descending sort
  unsigned* keys_sorted;
  int* vals;
  int* vals_sorted;
  unsigned char* keep;           // [V]
  void* sort_temp;
  size_t sort_temp_bytes;        // sample_sort_temp_bytes(V)
  float* scal;                   // [4]
  int* nkeep;
  float* argmax_v;               // [argmax_blocks()]
  int* argmax_i;
  // the drawn token
  int* out;
  int* seq;
  int* seq_len;
  int* pos_inc;
};
void sample(const SampleParams& p, hipStream_t s);
size_t sample_sort_temp_bytes(int V);
// Stable descending sort of n (key, value) pairs by key (equal keys keep
// their input order): keys_out / vals_out; vals null means the values are
// the indices 0..n-1. temp holds sample_sort_temp_bytes(n) bytes. Keys and
// the input are untouched; n <= kSortMax.
constexpr int kSortMax = 1 << 26;
void sort_pairs_desc(const unsigned* keys, const int* vals, int n, unsigned* keys_out, int* vals_out, void* temp,
                     hipStream_t s);

// ---------------------------------------------------------------- MoE --
// Router logits (bf16 GEMV), top-k with lowest-index ties, softmax over
// the k selected logits.
void moe_route(const float* xn, int T, const uint16_t* router, int E, int d, int k,
               int* sel, float* sel_w, hipStream_t s);

}  // namespace sg
