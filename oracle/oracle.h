/*
 * ORACLE — test infrastructure, not part of the product.
 *
 * A CPU (C + OpenMP) restatement of the StrasGPT reference forward pass,
 * used only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
 * leg, as the reference the HIP library's results are compared against and
 * as the timed CPU baseline.
 * The product (strasgpt_amd/) never links, loads or calls it.
 *
 * Every function restates one piece of the reference and cites it; the
 * per-element arithmetic (accumulation order of the bf16 dot product, fp32
 * RMSNorm, fp32 softmax attention, SwiGLU, RoPE table) follows the
 * reference source, while loop order and threading are free because each
 * output element is computed by one thread in a fixed order.
 *
 * Pins (see tests/test_oracle*.py):
 *  - bf16->f32 and MXFP4->f32: closed forms, exhaustive over all codes;
 *  - dot, rmsnorm, rope, attention, swiglu: float64 numpy restatements on
 *    small inputs, planted-mistake checks;
 *  - whole forward (dense): golden fixtures written by the reference C
 *    sources compiled into oracle/_ref (tokens identical, logits and
 *    normalised hidden states within 1e-4);
 *  - MoE router / experts: no reference counterpart; pinned by a float64
 *    numpy restatement of the defined semantics on tiny models (parity of
 *    the MoE path against the reference is unpinned by construction).
 */
#ifndef STRASGPT_ORACLE_H
#define STRASGPT_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ORACLE_CHUNK_MAX_LEN 512

typedef struct oracle_config {
  size_t embedding_dim, head_dim, hidden_dim, layer_count;
  size_t q_head_count, kv_head_count, vocabulary_len, context_len;
  float epsilon, rope_theta;
  int rope_interleaved;
  int qk_norm;
  int tied;                 /* out weight aliases the embedding */
  size_t expert_count;      /* 0: dense */
  size_t expert_used_count;
} oracle_config_t;

typedef struct oracle_model oracle_model_t;

/* Weight classes: the tensor kinds of the Hugging Face layout. */
enum {
  ORACLE_EMBEDDING, ORACLE_MHA_NORM, ORACLE_Q, ORACLE_Q_NORM, ORACLE_K,
  ORACLE_K_NORM, ORACLE_V, ORACLE_O, ORACLE_FFN_NORM, ORACLE_GATE, ORACLE_UP,
  ORACLE_DOWN, ORACLE_OUT_NORM, ORACLE_OUT, ORACLE_ROUTER,
  ORACLE_GATE_BLOCKS, ORACLE_GATE_SCALES, ORACLE_UP_BLOCKS, ORACLE_UP_SCALES,
  ORACLE_DOWN_BLOCKS, ORACLE_DOWN_SCALES, ORACLE_CLASS_COUNT
};

oracle_model_t* oracle_create(const oracle_config_t* cfg);
/* Reads size bytes at offset of file into weight class cls, layer. Returns
 * 0 on success, -1 on a size mismatch or I/O error. */
int oracle_load_tensor(oracle_model_t* m, int cls, size_t layer,
                       const char* file, size_t offset, size_t size);
/* Checks that every tensor was loaded; returns the number missing. */
int oracle_finalize(oracle_model_t* m);
void oracle_free(oracle_model_t* m);
void oracle_reset(oracle_model_t* m);
size_t oracle_cached_count(const oracle_model_t* m);
void oracle_set_threads(int n);

/* Reference transformer_predict (source/transformer.c:1607-1727). Returns
 * 0, or -1 when the context would overflow. */
int oracle_predict(oracle_model_t* m, size_t token_count, const int* token,
                   size_t logits_count, float* logits);
/* Capture for the next oracle_predict of T tokens (any count): residual
 * stream after every layer [L][T][d] and final-norm output [T][d]. */
void oracle_capture_hidden(oracle_model_t* m, float* out, float* out_final);
/* MoE models, for the next oracle_predict of T tokens: per layer and token
 * [L][T], the k-th largest router logit minus the largest one not selected
 * (0 for a tie at the cut; small values mean that another summation order
 * can select another expert set). No reference counterpart (the reference
 * has no MoE path). */
void oracle_capture_router_margin(oracle_model_t* m, float* out);

/* KV-cache storage formats (no reference counterpart: the reference cache
 * is fp32): every key and value row written to the cache (keys after their
 * norm and RoPE) is rounded to the format, round to nearest even, and read
 * back exactly by attention. */
enum { ORACLE_KV_F32 = 0, ORACLE_KV_BF16 = 1, ORACLE_KV_FP8_E4M3 = 2 };
void oracle_set_kv_format(oracle_model_t* m, int fmt);
float oracle_round_bf16(float x);
float oracle_round_fp8_e4m3(float x);

/* Reference sampler state (source/sampler.c:14-51, include/sampler.h:19-31)
 * and sampler_sample (source/sampler.c:234-337): presence penalty,
 * temperature, softmax, top-k, top-p, renormalization, multinomial draw
 * with the reference's xorshift64* coin. Equal probabilities rank by index
 * (a stable sort). coin_out gets the coin (-1 when greedy), margin_out the
 * distance from the coin to the sampled token's cdf interval ends and from
 * top_p to the top-p cutoff's cumulative sums (INFINITY when greedy). */
typedef struct {
  float temperature;
  size_t top_k;
  float top_p;
  float presence_penalty;
  unsigned long long rng_state;
} oracle_sampler_t;
size_t oracle_sample(oracle_sampler_t* s, float* logits, size_t n, unsigned char* presence,
                     int prev, float* coin_out, double* margin_out);

/* Reference sample_argmax (source/sampler.c:92-102). */
size_t oracle_argmax(const float* x, size_t n);

/* Primitive restatements, exported for unit pinning. */
float oracle_bf16_to_f32(uint16_t w);
/* The same over n codes into out (bit patterns kept, signaling NaNs included). */
void oracle_bf16_to_f32_array(const uint16_t* w, size_t n, float* out);
float oracle_mxfp4_value(uint8_t code, uint8_t scale);
void oracle_mxfp4_dequant(const uint8_t* blocks, const uint8_t* scales,
                          size_t value_count, float* out);
float oracle_dot_bf16(size_t len, const float* a, const uint16_t* w);
void oracle_rmsnorm(size_t n, float* y, const float* x, const uint16_t* w,
                    float eps);
void oracle_rope_table(size_t context_len, size_t head_dim, float theta,
                       int interleaved, float* out);
/* One query row against `count` cached keys/values: reference
 * source/transformer.c:1383-1419. */
void oracle_attention_row(size_t head_dim, size_t count, const float* q,
                          const float* k, const float* v, float* out);
void oracle_topk_softmax(size_t n, const float* logits, size_t k,
                         int* index, float* weight);

#ifdef __cplusplus
}
#endif

#endif
