/*
 * strasgpt-synth: writes a seeded random-init model directory that the
 * StrasGPT loader reads: config.json, model.safetensors (or shards plus
 * model.safetensors.index.json) and a minimal tokenizer.json.
 *
 * Values are a pure function of (seed, tensor name, element index) and are
 * produced with integer hashing plus correctly rounded double arithmetic
 * only, so every host writes bit-identical files:
 *   - bf16 matrices: Irwin-Hall(12) approximation of N(0, 1) scaled by the
 *     standard deviation (0.02 by default), rounded to bf16 (RNE);
 *   - norm weights (every "*norm.weight"): exactly 1.0;
 *   - MXFP4 "*_blocks": uniform bytes (two uniform E2M1 codes per byte);
 *   - MXFP4 "*_scales": uniform over E8M0 {119..123} = 2^-8 .. 2^-4.
 * Tensor names follow the Hugging Face layout that the reference loader
 * matches (reference include/safetensors.h:14-27).
 */
#define _GNU_SOURCE
#include <errno.h>
#include <omp.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>

#define DIE(...) do { fprintf(stderr, "[strasgpt-synth] error: " __VA_ARGS__); \
                      fprintf(stderr, "\n"); exit(EXIT_FAILURE); } while (0)

typedef enum { T_BF16, T_U8 } dtype_t;
typedef enum { V_NORMAL, V_ONE, V_BYTES, V_SCALES } vkind_t;

typedef struct {
  char name[160];
  dtype_t dtype;
  int ndim;
  size_t dim[4];
  vkind_t kind;
  size_t bytes;
  int shard;
  size_t begin; /* offset in the shard's data section */
} tdesc_t;

typedef struct {
  size_t dim, hidden, layers, heads, kv_heads, head_dim, vocab, ctx;
  size_t experts, experts_per_tok;
  double theta, eps, stddev;
  int qk_norm, untied, rope_interleaved, bos, eos;
  uint64_t seed;
  size_t shard_bytes;
  const char* out;
  const char* model_type;
} cfg_t;

static uint64_t mix64(uint64_t z) {
  z += 0x9E3779B97F4A7C15ull;
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

static uint64_t fnv1a64(const char* s) {
  uint64_t h = 0xCBF29CE484222325ull;
  for (; *s; s++) {
    h ^= (unsigned char)*s;
    h *= 0x100000001B3ull;
  }
  return h;
}

static uint16_t f32_to_bf16_rne(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  u += 0x7FFFu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

/* Irwin-Hall(12): sum of twelve 16-bit uniforms (centred in their cells),
 * minus 6: mean 0, variance 1 - 1/65536^2. */
static uint16_t normal_bf16(uint64_t key, size_t i, double stddev) {
  uint64_t s = 0;
  for (int r = 0; r < 3; r++) {
    uint64_t h = mix64(key + 3 * (uint64_t)i + (uint64_t)r);
    s += (h & 0xFFFF) + ((h >> 16) & 0xFFFF) + ((h >> 32) & 0xFFFF) + (h >> 48);
  }
  double z = ((double)s + 6.0) / 65536.0 - 6.0;
  return f32_to_bf16_rne((float)(z * stddev));
}

static void fill(const tdesc_t* t, uint64_t seed, double stddev, size_t first,
                 size_t count, uint8_t* out) {
  uint64_t key = mix64(seed ^ fnv1a64(t->name));
  if (t->dtype == T_BF16) {
    uint16_t* o = (uint16_t*)out;
    #pragma omp parallel for schedule(static)
    for (size_t j = 0; j < count; j++) {
      o[j] = t->kind == V_ONE ? 0x3F80 : normal_bf16(key, first + j, stddev);
    }
  } else {
    #pragma omp parallel for schedule(static)
    for (size_t j = 0; j < count; j++) {
      uint64_t h = mix64(key + first + j);
      out[j] = t->kind == V_SCALES ? (uint8_t)(119 + h % 5) : (uint8_t)(h >> 56);
    }
  }
}

static tdesc_t* add(tdesc_t* v, size_t* n, const char* name, dtype_t dt,
                    vkind_t kind, int ndim, size_t d0, size_t d1, size_t d2,
                    size_t d3) {
  tdesc_t* t = &v[(*n)++];
  memset(t, 0, sizeof(*t));
  snprintf(t->name, sizeof(t->name), "%s", name);
  t->dtype = dt;
  t->kind = kind;
  t->ndim = ndim;
  size_t d[4] = {d0, d1, d2, d3};
  size_t elems = 1;
  for (int i = 0; i < ndim; i++) {
    t->dim[i] = d[i];
    elems *= d[i];
  }
  t->bytes = elems * (dt == T_BF16 ? 2 : 1);
  return t;
}

static tdesc_t* build_table(const cfg_t* c, size_t* count) {
  size_t cap = 16 + c->layers * 16;
  tdesc_t* v = calloc(cap, sizeof(tdesc_t));
  size_t n = 0;
  char s[160];
  size_t d = c->dim, hd = c->head_dim, H = c->hidden, E = c->experts;
  add(v, &n, "model.embed_tokens.weight", T_BF16, V_NORMAL, 2, c->vocab, d, 0, 0);
  for (size_t l = 0; l < c->layers; l++) {
#define NAME(fmt) (snprintf(s, sizeof(s), fmt, l), s)
    add(v, &n, NAME("model.layers.%zu.input_layernorm.weight"), T_BF16, V_ONE, 1, d, 0, 0, 0);
    add(v, &n, NAME("model.layers.%zu.self_attn.q_proj.weight"), T_BF16, V_NORMAL, 2, c->heads * hd, d, 0, 0);
    add(v, &n, NAME("model.layers.%zu.self_attn.k_proj.weight"), T_BF16, V_NORMAL, 2, c->kv_heads * hd, d, 0, 0);
    add(v, &n, NAME("model.layers.%zu.self_attn.v_proj.weight"), T_BF16, V_NORMAL, 2, c->kv_heads * hd, d, 0, 0);
    add(v, &n, NAME("model.layers.%zu.self_attn.o_proj.weight"), T_BF16, V_NORMAL, 2, d, c->heads * hd, 0, 0);
    if (c->qk_norm) {
      add(v, &n, NAME("model.layers.%zu.self_attn.q_norm.weight"), T_BF16, V_ONE, 1, hd, 0, 0, 0);
      add(v, &n, NAME("model.layers.%zu.self_attn.k_norm.weight"), T_BF16, V_ONE, 1, hd, 0, 0, 0);
    }
    add(v, &n, NAME("model.layers.%zu.post_attention_layernorm.weight"), T_BF16, V_ONE, 1, d, 0, 0, 0);
    if (E == 0) {
      add(v, &n, NAME("model.layers.%zu.mlp.gate_proj.weight"), T_BF16, V_NORMAL, 2, H, d, 0, 0);
      add(v, &n, NAME("model.layers.%zu.mlp.up_proj.weight"), T_BF16, V_NORMAL, 2, H, d, 0, 0);
      add(v, &n, NAME("model.layers.%zu.mlp.down_proj.weight"), T_BF16, V_NORMAL, 2, d, H, 0, 0);
    } else {
      add(v, &n, NAME("model.layers.%zu.mlp.router.weight"), T_BF16, V_NORMAL, 2, E, d, 0, 0);
      add(v, &n, NAME("model.layers.%zu.mlp.experts.gate_proj_blocks"), T_U8, V_BYTES, 4, E, H, d / 32, 16);
      add(v, &n, NAME("model.layers.%zu.mlp.experts.gate_proj_scales"), T_U8, V_SCALES, 3, E, H, d / 32, 0);
      add(v, &n, NAME("model.layers.%zu.mlp.experts.up_proj_blocks"), T_U8, V_BYTES, 4, E, H, d / 32, 16);
      add(v, &n, NAME("model.layers.%zu.mlp.experts.up_proj_scales"), T_U8, V_SCALES, 3, E, H, d / 32, 0);
      add(v, &n, NAME("model.layers.%zu.mlp.experts.down_proj_blocks"), T_U8, V_BYTES, 4, E, d, H / 32, 16);
      add(v, &n, NAME("model.layers.%zu.mlp.experts.down_proj_scales"), T_U8, V_SCALES, 3, E, d, H / 32, 0);
    }
#undef NAME
  }
  add(v, &n, "model.norm.weight", T_BF16, V_ONE, 1, d, 0, 0, 0);
  if (c->untied) {
    add(v, &n, "lm_head.weight", T_BF16, V_NORMAL, 2, c->vocab, d, 0, 0);
  }
  *count = n;
  return v;
}

static void write_json_file(const char* path, const char* text) {
  FILE* f = fopen(path, "wb");
  if (!f) DIE("cannot create %s: %s", path, strerror(errno));
  fputs(text, f);
  fclose(f);
}

static char* header_json(tdesc_t* v, size_t n, int shard, size_t* len) {
  size_t cap = 256 + n * 256;
  char* h = malloc(cap);
  size_t p = 0;
  p += snprintf(h + p, cap - p, "{\"__metadata__\":{\"format\":\"pt\"}");
  for (size_t i = 0; i < n; i++) {
    if (v[i].shard != shard) continue;
    p += snprintf(h + p, cap - p, ",\"%s\":{\"dtype\":\"%s\",\"shape\":[",
                  v[i].name, v[i].dtype == T_BF16 ? "BF16" : "U8");
    for (int k = 0; k < v[i].ndim; k++) {
      p += snprintf(h + p, cap - p, "%s%zu", k ? "," : "", v[i].dim[k]);
    }
    p += snprintf(h + p, cap - p, "],\"data_offsets\":[%zu,%zu]}", v[i].begin,
                  v[i].begin + v[i].bytes);
  }
  p += snprintf(h + p, cap - p, "}");
  while (p % 8) h[p++] = ' '; /* data section starts 8-byte aligned */
  h[p] = 0;
  *len = p;
  return h;
}

int main(int argc, char** argv) {
  cfg_t c = {0};
  c.stddev = 0.02;
  c.eos = -1;
  c.bos = 0;
  c.model_type = "llama";
  for (int i = 1; i < argc; i++) {
    const char* a = argv[i];
    const char* v = i + 1 < argc ? argv[i + 1] : NULL;
#define ARG(flag) (strcmp(a, flag) == 0 && v && (i++, 1))
    if (ARG("--out")) c.out = v;
    else if (ARG("--seed")) c.seed = strtoull(v, 0, 10);
    else if (ARG("--dim")) c.dim = strtoull(v, 0, 10);
    else if (ARG("--hidden")) c.hidden = strtoull(v, 0, 10);
    else if (ARG("--layers")) c.layers = strtoull(v, 0, 10);
    else if (ARG("--heads")) c.heads = strtoull(v, 0, 10);
    else if (ARG("--kv-heads")) c.kv_heads = strtoull(v, 0, 10);
    else if (ARG("--head-dim")) c.head_dim = strtoull(v, 0, 10);
    else if (ARG("--vocab")) c.vocab = strtoull(v, 0, 10);
    else if (ARG("--ctx")) c.ctx = strtoull(v, 0, 10);
    else if (ARG("--theta")) c.theta = strtod(v, 0);
    else if (ARG("--eps")) c.eps = strtod(v, 0);
    else if (ARG("--std")) c.stddev = strtod(v, 0);
    else if (ARG("--experts")) c.experts = strtoull(v, 0, 10);
    else if (ARG("--experts-per-tok")) c.experts_per_tok = strtoull(v, 0, 10);
    else if (ARG("--shard-bytes")) c.shard_bytes = strtoull(v, 0, 10);
    else if (ARG("--model-type")) c.model_type = v;
    else if (ARG("--eos")) c.eos = atoi(v);
    else if (ARG("--threads")) omp_set_num_threads(atoi(v));
    else if (strcmp(a, "--qk-norm") == 0) c.qk_norm = 1;
    else if (strcmp(a, "--untied") == 0) c.untied = 1;
    else if (strcmp(a, "--rope-interleaved") == 0) c.rope_interleaved = 1;
    else DIE("unknown or incomplete argument %s", a);
#undef ARG
  }
  if (!c.out || !c.dim || !c.hidden || !c.layers || !c.heads || !c.kv_heads ||
      !c.head_dim || !c.vocab || !c.ctx)
    DIE("need --out --dim --hidden --layers --heads --kv-heads --head-dim --vocab --ctx");
  if (c.dim % 32 || c.hidden % 32) DIE("dim and hidden must be multiples of 32");
  if (c.experts && (!c.experts_per_tok || c.experts_per_tok > c.experts))
    DIE("bad --experts-per-tok");
  mkdir(c.out, 0755);

  size_t n;
  tdesc_t* v = build_table(&c, &n);
  int shards = 1;
  size_t acc = 0;
  for (size_t i = 0; i < n; i++) {
    if (c.shard_bytes && acc > 0 && acc + v[i].bytes > c.shard_bytes) {
      shards++;
      acc = 0;
    }
    v[i].shard = shards - 1;
    v[i].begin = acc;
    acc += (v[i].bytes + 7) / 8 * 8;
  }

  char path[4096];
  char* idx = NULL;
  size_t idx_cap = 0, idx_len = 0, idx_entries = 0;
  if (c.shard_bytes) {
    idx_cap = 256 + n * 256;
    idx = malloc(idx_cap);
    idx_len += snprintf(idx, idx_cap, "{\"metadata\":{\"total_size\":0},\"weight_map\":{");
  }
  size_t chunk_elems = 1 << 26;
  uint8_t* buf = malloc(chunk_elems * 2);
  for (int s = 0; s < shards; s++) {
    char fname[128];
    if (c.shard_bytes)
      snprintf(fname, sizeof(fname), "model-%05d-of-%05d.safetensors", s + 1, shards);
    else
      snprintf(fname, sizeof(fname), "model.safetensors");
    snprintf(path, sizeof(path), "%s/%s", c.out, fname);
    FILE* f = fopen(path, "wb");
    if (!f) DIE("cannot create %s: %s", path, strerror(errno));
    size_t hlen;
    char* h = header_json(v, n, s, &hlen);
    uint64_t hl = hlen;
    fwrite(&hl, 8, 1, f);
    fwrite(h, 1, hlen, f);
    free(h);
    for (size_t i = 0; i < n; i++) {
      if (v[i].shard != s) continue;
      size_t esz = v[i].dtype == T_BF16 ? 2 : 1;
      size_t elems = v[i].bytes / esz;
      for (size_t first = 0; first < elems; first += chunk_elems) {
        size_t cnt = elems - first < chunk_elems ? elems - first : chunk_elems;
        fill(&v[i], c.seed, c.stddev, first, cnt, buf);
        if (fwrite(buf, esz, cnt, f) != cnt) DIE("short write to %s", path);
      }
      static const char zeros[8] = {0};
      size_t pad = (8 - v[i].bytes % 8) % 8;
      if (pad) fwrite(zeros, 1, pad, f);
      if (idx) {
        idx_len += snprintf(idx + idx_len, idx_cap - idx_len, "%s\"%s\":\"%s\"",
                            idx_entries++ ? "," : "", v[i].name, fname);
      }
    }
    if (fclose(f) != 0) DIE("close failed on %s", path);
  }
  free(buf);
  if (idx) {
    snprintf(idx + idx_len, idx_cap - idx_len, "}}\n");
    snprintf(path, sizeof(path), "%s/model.safetensors.index.json", c.out);
    write_json_file(path, idx);
    free(idx);
  }

  char cfgtxt[4096];
  int p = snprintf(cfgtxt, sizeof(cfgtxt),
      "{\n  \"architectures\": [\"%s\"],\n  \"model_type\": \"%s\",\n"
      "  \"hidden_size\": %zu,\n  \"intermediate_size\": %zu,\n"
      "  \"num_hidden_layers\": %zu,\n  \"num_attention_heads\": %zu,\n"
      "  \"num_key_value_heads\": %zu,\n  \"head_dim\": %zu,\n"
      "  \"vocab_size\": %zu,\n  \"max_position_embeddings\": %zu,\n"
      "  \"rms_norm_eps\": %.9g,\n  \"rope_theta\": %.1f,\n"
      "  \"rope_scaling\": %s,\n"
      "  \"bos_token_id\": %d,\n  \"eos_token_id\": %d,\n"
      "  \"tie_word_embeddings\": %s,\n  \"torch_dtype\": \"bfloat16\"",
      c.experts ? "StrasMoeForCausalLM" : "LlamaForCausalLM", c.model_type,
      c.dim, c.hidden, c.layers, c.heads, c.kv_heads, c.head_dim, c.vocab,
      c.ctx, c.eps, c.theta,
      c.rope_interleaved ? "{\"mrope_interleaved\": true}" : "null",
      c.bos, c.eos, c.untied ? "false" : "true");
  if (c.experts)
    p += snprintf(cfgtxt + p, sizeof(cfgtxt) - p,
                  ",\n  \"num_local_experts\": %zu,\n  \"num_experts_per_tok\": %zu",
                  c.experts, c.experts_per_tok);
  snprintf(cfgtxt + p, sizeof(cfgtxt) - p, "\n}\n");
  snprintf(path, sizeof(path), "%s/config.json", c.out);
  write_json_file(path, cfgtxt);

  /* Minimal tokenizer.json: the reference driver loads one even with
   * --pre-tokenized; token i is the string "<i>". */
  snprintf(path, sizeof(path), "%s/tokenizer.json", c.out);
  FILE* f = fopen(path, "wb");
  if (!f) DIE("cannot create %s", path);
  fprintf(f, "{\"model\":{\"type\":\"BPE\",\"vocab\":{");
  for (size_t i = 0; i < c.vocab; i++) fprintf(f, "%s\"<%zu>\":%zu", i ? "," : "", i, i);
  fprintf(f, "}}}\n");
  fclose(f);
  free(v);
  return 0;
}
