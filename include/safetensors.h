/*
 * Model description read from a Hugging Face model directory: config.json,
 * optional model.safetensors.index.json, and one or more .safetensors files.
 *
 * Drop-in replacement for the reference loader (include/safetensors.h and
 * source/safetensors.c of StrasGPT). The struct layout of safetensors_t and
 * safetensors_tensor_t is kept field-for-field identical to the reference
 * (include/safetensors.h:43-81) so that a caller compiled against the
 * reference header can hand its safetensors_t to this library. Additions
 * live strictly after the reference fields:
 *   - dtype U8 (value 3) for MXFP4 expert blocks/scales; the reference only
 *     knows F16/BF16/F32 and dies on anything else
 *     (source/safetensors.c:365-378);
 *   - MoE hyper-parameters appended after the tensor table; they are only
 *     read when MoE tensors are present, which the reference parser can
 *     never produce (it dies on dtype U8).
 */
#ifndef SAFETENSORS_H
# define SAFETENSORS_H

#include <stdbool.h>
#include <stddef.h>
#include <stdio.h>

#ifdef __cplusplus
extern "C" {
#endif

struct options;

#define SAFETENSORS_FILE_CONFIG      "config.json"
#define SAFETENSORS_FILE_INDEX       "model.safetensors.index.json"
#define SAFETENSORS_FILE_SAFETENSORS "model.safetensors"

/* Hugging Face tensor names (a file format: identical to the reference,
 * include/safetensors.h:14-27). "%d" is the layer index. */
#define SAFETENSORS_PATTERN_EMBEDDING_WEIGHT  "model.embed_tokens.weight"
#define SAFETENSORS_PATTERN_MHA_NORM_WEIGHT   "model.layers.%d.input_layernorm.weight"
#define SAFETENSORS_PATTERN_MHA_Q_WEIGHT      "model.layers.%d.self_attn.q_proj.weight"
#define SAFETENSORS_PATTERN_MHA_Q_NORM_WEIGHT "model.layers.%d.self_attn.q_norm.weight"
#define SAFETENSORS_PATTERN_MHA_K_WEIGHT      "model.layers.%d.self_attn.k_proj.weight"
#define SAFETENSORS_PATTERN_MHA_K_NORM_WEIGHT "model.layers.%d.self_attn.k_norm.weight"
#define SAFETENSORS_PATTERN_MHA_V_WEIGHT      "model.layers.%d.self_attn.v_proj.weight"
#define SAFETENSORS_PATTERN_MHA_OUT_WEIGHT    "model.layers.%d.self_attn.o_proj.weight"
#define SAFETENSORS_PATTERN_FFN_NORM_WEIGHT   "model.layers.%d.post_attention_layernorm.weight"
#define SAFETENSORS_PATTERN_FFN_FC_WEIGHT     "model.layers.%d.mlp.gate_proj.weight"
#define SAFETENSORS_PATTERN_FFN_UP_WEIGHT     "model.layers.%d.mlp.up_proj.weight"
#define SAFETENSORS_PATTERN_FFN_OUT_WEIGHT    "model.layers.%d.mlp.down_proj.weight"
#define SAFETENSORS_PATTERN_OUT_NORM_WEIGHT   "model.norm.weight"
#define SAFETENSORS_PATTERN_OUT_WEIGHT        "lm_head.weight"

/* MXFP4 mixture-of-experts tensors (no reference counterpart). Expert
 * matrices are stored gpt-oss style: "<name>_blocks" U8 [E][N][K/32][16]
 * holds two E2M1 codes per byte (element 2j in the low nibble), and
 * "<name>_scales" U8 [E][N][K/32] holds one E8M0 exponent per 32 values. */
#define SAFETENSORS_PATTERN_MOE_ROUTER_WEIGHT "model.layers.%d.mlp.router.weight"
#define SAFETENSORS_PATTERN_MOE_GATE_BLOCKS   "model.layers.%d.mlp.experts.gate_proj_blocks"
#define SAFETENSORS_PATTERN_MOE_GATE_SCALES   "model.layers.%d.mlp.experts.gate_proj_scales"
#define SAFETENSORS_PATTERN_MOE_UP_BLOCKS     "model.layers.%d.mlp.experts.up_proj_blocks"
#define SAFETENSORS_PATTERN_MOE_UP_SCALES     "model.layers.%d.mlp.experts.up_proj_scales"
#define SAFETENSORS_PATTERN_MOE_DOWN_BLOCKS   "model.layers.%d.mlp.experts.down_proj_blocks"
#define SAFETENSORS_PATTERN_MOE_DOWN_SCALES   "model.layers.%d.mlp.experts.down_proj_scales"

#define SAFETENSORS_MAX_FILE_COUNT          64
#define SAFETENSORS_MAX_DIM_COUNT           8
#define SAFETENSORS_MAX_MROPE_SECTION_COUNT 8
#define SAFETENSORS_MAX_TENSOR_COUNT        65536
#define SAFETENSORS_MAX_STRING              1024

typedef enum {
  SAFETENSORS_TYPE_F16,  /* IEEE binary16 */
  SAFETENSORS_TYPE_BF16, /* bfloat16 */
  SAFETENSORS_TYPE_F32,  /* IEEE binary32 */
  SAFETENSORS_TYPE_U8    /* raw bytes (MXFP4 blocks and scales) */
} safetensors_type_t;

extern const char* safetensors_type_str[];

typedef struct safetensors_tensor_t {
  char* name;
  safetensors_type_t type;
  size_t dim_count;
  size_t dim[SAFETENSORS_MAX_DIM_COUNT];
  size_t size;   /* bytes */
  size_t file;   /* index into safetensors_t.file */
  size_t offset; /* absolute byte offset of the data in that file */
} safetensors_tensor_t;

typedef struct safetensors {
  /* --- fields of the reference struct, same order and types --- */
  char* model_type;
  size_t embedding_dim;  /* hidden_size */
  size_t head_dim;       /* head_dim (default hidden_size / heads) */
  size_t hidden_dim;     /* intermediate_size */
  size_t layer_count;    /* num_hidden_layers */
  size_t q_head_count;   /* num_attention_heads */
  size_t kv_head_count;  /* num_key_value_heads */
  size_t vocabulary_len; /* vocab_size */
  size_t context_len;    /* max_position_embeddings */
  float epsilon;         /* rms_norm_eps */
  float rope_theta;      /* rope_theta */
  bool rope_interleaved; /* rope_scaling.mrope_interleaved */
  size_t mrope_section_count;
  size_t mrope_section[SAFETENSORS_MAX_MROPE_SECTION_COUNT];
  int bos_token_id;
  int eos_token_id;
  size_t file_count;
  char* file[SAFETENSORS_MAX_FILE_COUNT];
  size_t tensor_count;
  safetensors_tensor_t tensor[SAFETENSORS_MAX_TENSOR_COUNT];
  /* --- additions (absent from the reference struct) --- */
  size_t expert_count;      /* num_local_experts (0: dense model) */
  size_t expert_used_count; /* num_experts_per_tok */
} safetensors_t;

safetensors_t* safetensors_malloc(void);
void safetensors_free(safetensors_t* safetensors);
void safetensors_print(FILE* f, const safetensors_t* safetensors);
void safetensors_print_model_infos(FILE* f, const safetensors_t* s);
/* Reads options->model_dir (struct options of the reference driver: the
 * model_dir field is read through safetensors_options_model_dir). */
safetensors_t* safetensors_read(struct options* options);
safetensors_type_t safetensors_type_from_string(const char* s);
void safetensors_file_lookup(safetensors_t* s, char* path, char* file);
size_t safetensors_sizeof(safetensors_type_t type);
bool safetensors_aliased_out_weight(const safetensors_t* safetensors);

/* Addition: read a model directory given by path (what safetensors_read
 * does with options->model_dir, reference source/json_parser.y:526-622). */
safetensors_t* safetensors_read_dir(const char* model_dir);

/* The JSON front-end's scanner cleanup, called by the reference driver at
 * exit (reference source/strasgpt.c:30,287; flex-generated in the
 * reference, source/json_scanner.l). The library's reader holds no scanner
 * state, so it frees nothing; it exists so that the reference driver links
 * against the library with its lex/yacc front-end removed. Returns 0. */
int json_scanner_lex_destroy(void);

#ifdef __cplusplus
}
#endif

#endif /* SAFETENSORS_H */
