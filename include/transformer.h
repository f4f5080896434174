/*
 * StrasGPT transformer forward pass on one AMD Instinct MI355X (gfx950).
 *
 * Drop-in replacement for the reference C API (include/transformer.h:87-99
 * of StrasGPT). The five entry points keep their names, argument meaning
 * and error behaviour (print "[StrasGPT] Error ..." and exit on failure).
 * transformer_configuration_t keeps the reference layout (callers read
 * config->vocabulary_len, reference source/sampler.c:27); fields after
 * aliased_out_weight are additions. transformer_weights_t and
 * transformer_state_t hold DEVICE pointers (HBM) here: callers never
 * dereference them in the reference driver.
 *
 * Threading: like the reference, transformer_predict may be called by
 * every thread of an OpenMP team (reference source/strasgpt.c:209-232).
 * One thread does the device work; every thread returns only once the
 * logits are in the caller's buffer. It also works outside a parallel
 * region.
 */
#ifndef TRANSFORMER_H
# define TRANSFORMER_H

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>
#include <stdio.h>

#ifdef __cplusplus
extern "C" {
#endif

struct safetensors;

/* Reference include/transformer.h:9: prefill is processed in chunks of at
 * most this many tokens. */
#define TRANSFORMER_CHUNK_MAX_LEN 512

typedef struct transformer_configuration {
  size_t embedding_dim;
  size_t head_dim;
  size_t hidden_dim;       /* dense FFN width, or expert FFN width (MoE) */
  size_t layer_count;
  size_t q_head_count;
  size_t kv_head_count;
  size_t vocabulary_len;
  size_t context_len;
  float epsilon;
  float rope_theta;
  size_t rope_pair_bound;  /* interleaved: head_dim, half-split: head_dim/2 */
  size_t rope_pair_offset; /* interleaved: 1,        half-split: head_dim/2 */
  size_t rope_pair_stride; /* interleaved: 2,        half-split: 1 */
  size_t mrope_section_count;
  size_t* mrope_section;
  bool aliased_out_weight;
  /* --- additions --- */
  bool qk_norm;             /* per-head q/k RMSNorm present */
  size_t expert_count;      /* 0 for dense models */
  size_t expert_used_count; /* experts per token (top-k) */
} transformer_configuration_t;

/* Device (HBM) weight pointers. Dense layout per layer is the Hugging Face
 * row-major [out][in] bf16 layout; Q, K and V rows are stored fused per
 * layer as one [(q_heads + 2*kv_heads) * head_dim][embedding_dim] matrix.
 * MXFP4 experts keep their [E][N][K/32][16] code bytes and [E][N][K/32]
 * exponents. */
typedef struct transformer_weights {
  uint16_t* embedding_weight;  /* [vocabulary_len][embedding_dim] */
  uint16_t* mha_norm_weight;   /* [layer_count][embedding_dim] */
  uint16_t* mha_qkv_weight;    /* [layer_count][(qh+2kvh)*head_dim][embedding_dim] */
  uint16_t* mha_q_norm_weight; /* [layer_count][head_dim] or NULL */
  uint16_t* mha_k_norm_weight; /* [layer_count][head_dim] or NULL */
  uint16_t* mha_out_weight;    /* [layer_count][embedding_dim][qh*head_dim] */
  uint16_t* ffn_norm_weight;   /* [layer_count][embedding_dim] */
  uint16_t* ffn_fc_weight;     /* [layer_count][hidden_dim][embedding_dim] */
  uint16_t* ffn_up_weight;     /* [layer_count][hidden_dim][embedding_dim] */
  uint16_t* ffn_out_weight;    /* [layer_count][embedding_dim][hidden_dim] */
  uint16_t* out_norm_weight;   /* [embedding_dim] */
  uint16_t* out_weight;        /* [vocabulary_len][embedding_dim] (may alias) */
  /* MoE (NULL for dense models) */
  uint16_t* moe_router_weight; /* [layer_count][expert_count][embedding_dim] */
  uint8_t* moe_gate_blocks;    /* [layer_count][E][hidden_dim][embedding_dim/2] */
  uint8_t* moe_gate_scales;    /* [layer_count][E][hidden_dim][embedding_dim/32] */
  uint8_t* moe_up_blocks;
  uint8_t* moe_up_scales;
  uint8_t* moe_down_blocks;    /* [layer_count][E][embedding_dim][hidden_dim/2] */
  uint8_t* moe_down_scales;    /* [layer_count][E][embedding_dim][hidden_dim/32] */
} transformer_weights_t;

/* Device (HBM) activation state. */
typedef struct transformer_state {
  float* embedding;    /* [chunk][embedding_dim] residual stream */
  float* mha_q;        /* [chunk][q_head_count*head_dim] */
  float* mha_att;      /* [chunk][q_head_count*head_dim] */
  float* ffn_act;      /* [chunk][hidden_dim] SwiGLU output */
  float* logits;       /* [chunk][vocabulary_len] */
  size_t cached_count; /* positions held in the KV cache */
  float* k_cache;      /* [layer_count][kv_head_count][context_len][head_dim] */
  float* v_cache;      /* [layer_count][kv_head_count][context_len][head_dim] */
  float* rope_cos_sin; /* [context_len][head_dim] */
} transformer_state_t;

struct transformer_device;

typedef struct transformer {
  transformer_configuration_t* config;
  transformer_weights_t* weights;
  transformer_state_t* state;
  struct transformer_device* device; /* addition: opaque runtime context */
} transformer_t;

/* Reference include/transformer.h:87. Uploads every tensor once to HBM. */
transformer_t* transformer_from_safetensors(struct safetensors* safetensors);
/* Reference include/transformer.h:88. NULL-safe. */
void transformer_free(transformer_t* transformer);
/* Reference include/transformer.h:89. Summaries come from host copies made
 * at upload time; device memory is never read here. */
void transformer_print(FILE* f, const transformer_t* transformer);
/* Reference include/transformer.h:90-92. Plain malloc: free() it. */
float* transformer_logits_malloc(
    transformer_t* transformer, size_t logits_count, size_t* vocabulary_len
);
/* Reference include/transformer.h:93-99. Appends token_count positions to
 * the KV cache and writes fp32 logits of the last min(logits_count,
 * token_count) positions, row-major [row][vocabulary_len]. Returns silently
 * if transformer or logits is NULL or a count is 0; exits with
 * "context length exhausted" when the cache would overflow. Synchronous. */
void transformer_predict(
    transformer_t* transformer,
    size_t token_count,
    int* token,
    size_t logits_count,
    float* logits
);

#ifdef __cplusplus
}
#endif

#endif /* TRANSFORMER_H */
