/*
 * Safetensors model-directory loader: config.json, optional
 * model.safetensors.index.json, and each .safetensors header.
 *
 * The reference generates its parser with lex/yacc (source/json_parser.y,
 * source/json_scanner.l); this is a hand-written recursive-descent reader
 * with the same key semantics:
 *  - config keys and their meaning: json_scanner.l:27-50 and
 *    json_parser.y:71-244 (integer keys reject non-integral numbers,
 *    rms_norm_eps / rope_theta take any number, rope_scaling may be null or
 *    an object whose mrope_section / mrope_interleaved members are read,
 *    text_config nests a second config object, unknown keys are skipped);
 *  - index.json: files listed in order of first appearance in weight_map
 *    (json_parser.y:250-277, safetensors.c:381-403);
 *  - tensor byte range: offset = 8 + header_len + begin, size = end - begin
 *    (json_parser.y:327-338);
 *  - head_dim defaults to hidden_size / num_attention_heads
 *    (json_parser.y:616-619).
 * tokenizer.json (json_parser.y:380-446, 626-648): the entries of the
 * top-level "model" object's "vocab" object, key bytes as written and the
 * number as a float score, in file order; other members are skipped.
 * Differences, all additive: dtype "U8" is accepted (MXFP4 tensors),
 * num_local_experts / num_experts_per_tok are read, and an array-valued
 * bos/eos_token_id takes its first element (the reference rejects arrays).
 */
#define _GNU_SOURCE
#include "safetensors.h"

#include <limits.h>
#include <math.h>
#include <stdint.h>
#include <string.h>

#include "common.h"
#include "tokenizer.h"

const char* safetensors_type_str[] = {"F16", "BF16", "F32", "U8"};

safetensors_t* safetensors_malloc(void) {
  safetensors_t* s = calloc(1, sizeof(safetensors_t));
  if (!s) ST_DIE("failed to malloc for safetensors_t");
  return s;
}

void safetensors_free(safetensors_t* s) {
  if (!s) return;
  free(s->model_type);
  for (size_t i = 0; i < s->file_count; i++) free(s->file[i]);
  for (size_t i = 0; i < s->tensor_count; i++) free(s->tensor[i].name);
  free(s);
}

static char* read_file(const char* path, size_t* len, bool required);
static char* read_file_optional(const char* path, size_t* len) { return read_file(path, len, false); }

/* ------------------------------------------------------------------------ */
/* Minimal JSON reader                                                       */

typedef struct {
  const char* p;
  const char* end;
  const char* what; /* file being read, for messages */
  size_t line;
} json_t;

typedef struct {
  bool is_int;
  long long ival;
  double fval;
} number_t;

static void json_fail(json_t* j, const char* msg) {
  char m[SAFETENSORS_MAX_STRING];
  snprintf(m, sizeof(m), "%s: line %zu: %s", j->what, j->line, msg);
  ST_ERROR(m);
}

static void json_ws(json_t* j) {
  while (j->p < j->end) {
    char c = *j->p;
    if (c == '\n') j->line++;
    if (c == ' ' || c == '\t' || c == '\n' || c == '\r') j->p++;
    else break;
  }
}

static int json_peek(json_t* j) {
  json_ws(j);
  return j->p < j->end ? (unsigned char)*j->p : -1;
}

static void json_expect(json_t* j, char c) {
  if (json_peek(j) != c) {
    char m[64];
    snprintf(m, sizeof(m), "syntax error (expected '%c')", c);
    json_fail(j, m);
  }
  j->p++;
}

/* Returns the raw characters between the quotes (escape sequences are kept
 * verbatim, as the reference scanner does). */
static char* json_string(json_t* j) {
  json_expect(j, '"');
  const char* start = j->p;
  while (j->p < j->end && *j->p != '"') {
    if (*j->p == '\\' && j->p + 1 < j->end) j->p++;
    if (*j->p == '\n') j->line++;
    j->p++;
  }
  if (j->p >= j->end) json_fail(j, "unterminated string");
  size_t n = (size_t)(j->p - start);
  char* s = malloc(n + 1);
  if (!s) ST_DIE("malloc failed for string");
  memcpy(s, start, n);
  s[n] = 0;
  j->p++;
  return s;
}

static number_t json_number(json_t* j) {
  json_ws(j);
  const char* s = j->p;
  bool is_float = false;
  if (j->p < j->end && (*j->p == '+' || *j->p == '-')) j->p++;
  while (j->p < j->end) {
    char c = *j->p;
    if (c >= '0' && c <= '9') j->p++;
    else if (c == '.' || c == 'e' || c == 'E' ||
             ((c == '+' || c == '-') && (j->p[-1] == 'e' || j->p[-1] == 'E'))) {
      is_float = true;
      j->p++;
    } else break;
  }
  if (j->p == s) json_fail(j, "syntax error (expected a number)");
  char buf[128];
  size_t n = (size_t)(j->p - s);
  if (n >= sizeof(buf)) json_fail(j, "number too long");
  memcpy(buf, s, n);
  buf[n] = 0;
  number_t v;
  if (!is_float) {
    v.is_int = true;
    v.ival = atoll(buf);
    v.fval = (double)v.ival;
  } else {
    v.fval = atof(buf);
    double ip;
    v.is_int = modf(v.fval, &ip) == 0.0 && v.fval >= (double)LLONG_MIN &&
               v.fval <= (double)LLONG_MAX;
    v.ival = v.is_int ? (long long)v.fval : 0;
  }
  return v;
}

static bool json_literal(json_t* j, const char* lit) {
  size_t n = strlen(lit);
  json_ws(j);
  if ((size_t)(j->end - j->p) >= n && memcmp(j->p, lit, n) == 0) {
    j->p += n;
    return true;
  }
  return false;
}

static void json_skip(json_t* j) {
  int c = json_peek(j);
  if (c == '"') {
    free(json_string(j));
  } else if (c == '{' || c == '[') {
    char close = c == '{' ? '}' : ']';
    j->p++;
    if (json_peek(j) == close) {
      j->p++;
      return;
    }
    for (;;) {
      if (c == '{') {
        free(json_string(j));
        json_expect(j, ':');
      }
      json_skip(j);
      int d = json_peek(j);
      if (d == ',') {
        j->p++;
        continue;
      }
      json_expect(j, close);
      return;
    }
  } else if (json_literal(j, "true") || json_literal(j, "false") ||
             json_literal(j, "null")) {
    return;
  } else {
    (void)json_number(j);
  }
}

/* Iterates over the members of an object: calls member(key) with the
 * reader positioned on the value; member must consume the value. */
typedef void (*member_fn)(json_t* j, const char* key, void* ctx);

static void json_object(json_t* j, member_fn member, void* ctx) {
  json_expect(j, '{');
  if (json_peek(j) == '}') {
    j->p++;
    return;
  }
  for (;;) {
    char* key = json_string(j);
    json_expect(j, ':');
    member(j, key, ctx);
    free(key);
    int c = json_peek(j);
    if (c == ',') {
      j->p++;
      continue;
    }
    json_expect(j, '}');
    return;
  }
}

static size_t json_size(json_t* j, const char* key) {
  number_t n = json_number(j);
  if (!n.is_int || n.ival < 0) {
    char m[128];
    snprintf(m, sizeof(m), "non integer %s value", key);
    json_fail(j, m);
  }
  return (size_t)n.ival;
}

static int json_token_id(json_t* j, const char* key) {
  if (json_peek(j) == '[') {
    j->p++;
    int v = -1;
    bool first = true;
    while (json_peek(j) != ']') {
      number_t n = json_number(j);
      if (!n.is_int) json_fail(j, "non integer token id");
      if (first) v = (int)n.ival;
      first = false;
      if (json_peek(j) == ',') j->p++;
    }
    j->p++;
    return v;
  }
  number_t n = json_number(j);
  if (!n.is_int) {
    char m[128];
    snprintf(m, sizeof(m), "non integer %s", key);
    json_fail(j, m);
  }
  return (int)n.ival;
}

/* ------------------------------------------------------------------------ */
/* config.json                                                               */

static void rope_scaling_member(json_t* j, const char* key, void* ctx) {
  safetensors_t* s = ctx;
  if (strcmp(key, "mrope_section") == 0) {
    json_expect(j, '[');
    while (json_peek(j) != ']') {
      number_t n = json_number(j);
      if (!n.is_int) json_fail(j, "non integer mrope section value");
      if (s->mrope_section_count >= SAFETENSORS_MAX_MROPE_SECTION_COUNT)
        json_fail(j, "too many mrope sections");
      s->mrope_section[s->mrope_section_count++] = (size_t)n.ival;
      if (json_peek(j) == ',') j->p++;
    }
    j->p++;
  } else if (strcmp(key, "mrope_interleaved") == 0) {
    if (json_literal(j, "true")) s->rope_interleaved = true;
    else if (json_literal(j, "false")) s->rope_interleaved = false;
    else json_fail(j, "syntax error (expected a boolean)");
  } else {
    json_skip(j);
  }
}

static void config_member(json_t* j, const char* key, void* ctx) {
  safetensors_t* s = ctx;
  if (json_peek(j) == 'n' && strcmp(key, "rope_scaling") != 0) {
    json_skip(j); /* null value: key not set */
    return;
  }
  if (strcmp(key, "bos_token_id") == 0) s->bos_token_id = json_token_id(j, key);
  else if (strcmp(key, "eos_token_id") == 0) s->eos_token_id = json_token_id(j, key);
  else if (strcmp(key, "hidden_size") == 0) s->embedding_dim = json_size(j, key);
  else if (strcmp(key, "head_dim") == 0) s->head_dim = json_size(j, key);
  else if (strcmp(key, "intermediate_size") == 0) s->hidden_dim = json_size(j, key);
  else if (strcmp(key, "num_hidden_layers") == 0) s->layer_count = json_size(j, key);
  else if (strcmp(key, "num_attention_heads") == 0) s->q_head_count = json_size(j, key);
  else if (strcmp(key, "num_key_value_heads") == 0) s->kv_head_count = json_size(j, key);
  else if (strcmp(key, "vocab_size") == 0) s->vocabulary_len = json_size(j, key);
  else if (strcmp(key, "max_position_embeddings") == 0) s->context_len = json_size(j, key);
  else if (strcmp(key, "num_local_experts") == 0) s->expert_count = json_size(j, key);
  else if (strcmp(key, "num_experts_per_tok") == 0) s->expert_used_count = json_size(j, key);
  else if (strcmp(key, "rms_norm_eps") == 0) s->epsilon = (float)json_number(j).fval;
  else if (strcmp(key, "rope_theta") == 0) s->rope_theta = (float)json_number(j).fval;
  else if (strcmp(key, "model_type") == 0) {
    free(s->model_type);
    s->model_type = json_string(j);
  } else if (strcmp(key, "rope_scaling") == 0) {
    if (json_peek(j) == '{') json_object(j, rope_scaling_member, s);
    else if (!json_literal(j, "null")) json_fail(j, "syntax error in rope_scaling");
  } else if (strcmp(key, "text_config") == 0) {
    json_object(j, config_member, s);
  } else {
    json_skip(j);
  }
}

/* ------------------------------------------------------------------------ */
/* model.safetensors.index.json                                              */

typedef struct {
  safetensors_t* s;
  const char* dir;
} index_ctx_t;

static void weight_map_member(json_t* j, const char* key, void* ctx) {
  (void)key;
  index_ctx_t* c = ctx;
  char* file = json_string(j);
  safetensors_file_lookup(c->s, (char*)c->dir, file);
  free(file);
}

static void index_member(json_t* j, const char* key, void* ctx) {
  if (strcmp(key, "weight_map") == 0) json_object(j, weight_map_member, ctx);
  else json_skip(j);
}

/* ------------------------------------------------------------------------ */
/* .safetensors header                                                       */

typedef struct {
  safetensors_t* s;
  size_t file;
  size_t header_len;
  safetensors_tensor_t* t;
} header_ctx_t;

static void tensor_member(json_t* j, const char* key, void* ctx) {
  header_ctx_t* c = ctx;
  safetensors_tensor_t* t = c->t;
  if (strcmp(key, "dtype") == 0) {
    char* d = json_string(j);
    t->type = safetensors_type_from_string(d);
    free(d);
  } else if (strcmp(key, "shape") == 0) {
    json_expect(j, '[');
    t->dim_count = 0;
    while (json_peek(j) != ']') {
      number_t n = json_number(j);
      if (!n.is_int) json_fail(j, "non integer dimension value");
      if (t->dim_count >= SAFETENSORS_MAX_DIM_COUNT)
        json_fail(j, "too many tensor dimensions");
      t->dim[t->dim_count++] = (size_t)n.ival;
      if (json_peek(j) == ',') j->p++;
    }
    j->p++;
  } else if (strcmp(key, "data_offsets") == 0) {
    json_expect(j, '[');
    number_t b = json_number(j);
    json_expect(j, ',');
    number_t e = json_number(j);
    json_expect(j, ']');
    if (!b.is_int || !e.is_int) json_fail(j, "non integer offset value");
    if (e.ival < b.ival || b.ival < 0) json_fail(j, "bad data_offsets");
    t->size = (size_t)(e.ival - b.ival);
    t->offset = 8 + c->header_len + (size_t)b.ival;
    t->file = c->file;
  } else {
    json_skip(j);
  }
}

static void header_member(json_t* j, const char* key, void* ctx) {
  header_ctx_t* c = ctx;
  if (strcmp(key, "__metadata__") == 0 || strcmp(key, "metadata") == 0) {
    json_skip(j);
    return;
  }
  if (c->s->tensor_count >= SAFETENSORS_MAX_TENSOR_COUNT)
    json_fail(j, "too many tensors");
  safetensors_tensor_t* t = &c->s->tensor[c->s->tensor_count];
  memset(t, 0, sizeof(*t));
  c->t = t;
  json_object(j, tensor_member, c);
  t->name = strdup(key);
  c->s->tensor_count++;
}

/* ------------------------------------------------------------------------ */
/* tokenizer.json                                                            */

/* Entries of model.vocab in file order (reference json_parser.y:404-446):
 * key bytes as written, the number as the score. */
static void vocab_member(json_t* j, const char* key, void* ctx) {
  tokenizer_t* t = ctx;
  if (t->token_string_count >= TOKENIZER_MAX_TOKEN_STRING) json_fail(j, "too many token strings");
  number_t n = json_number(j);
  char* copy = strdup(key);
  if (!copy) ST_DIE("malloc failed for token string");
  t->token_string[t->token_string_count] = copy;
  t->score[t->token_string_count] = (float)n.fval;
  t->token_string_count++;
}

static void tokenizer_model_member(json_t* j, const char* key, void* ctx) {
  if (strcmp(key, "vocab") != 0) {
    json_skip(j);
    return;
  }
  tokenizer_t* t = ctx;
  size_t before = t->token_string_count;
  json_object(j, vocab_member, t);
  /* the reference grammar has no empty vocab object (json_parser.y:431) */
  if (t->token_string_count == before) json_fail(j, "syntax error (empty vocab)");
}

static void tokenizer_member(json_t* j, const char* key, void* ctx) {
  if (strcmp(key, "model") != 0) {
    json_skip(j);
    return;
  }
  if (json_peek(j) != '{') json_fail(j, "syntax error (model is not an object)");
  json_object(j, tokenizer_model_member, ctx);
}

void st_read_tokenizer_json(const char* path, tokenizer_t* t) {
  size_t len;
  char* text = read_file_optional(path, &len);
  if (!text) ST_DIE("failed to open tokenizer file");
  json_t j = {text, text + len, TOKENIZER_FILE, 1};
  json_object(&j, tokenizer_member, t);
  free(text);
}

/* ------------------------------------------------------------------------ */

static char* read_file(const char* path, size_t* len, bool required) {
  FILE* f = fopen(path, "rb");
  if (!f) {
    if (!required) return NULL;
    fprintf(stderr, "[StrasGPT] Error: failed to open file %s\n", path);
    fprintf(stderr, "Use \"-m <path_to_model_directory>\" option\n");
    exit(EXIT_FAILURE);
  }
  fseek(f, 0, SEEK_END);
  long n = ftell(f);
  fseek(f, 0, SEEK_SET);
  char* buf = malloc((size_t)n + 1);
  if (!buf) ST_DIE("malloc failed for file buffer");
  if (fread(buf, 1, (size_t)n, f) != (size_t)n) ST_DIE("failed to read file");
  fclose(f);
  buf[n] = 0;
  *len = (size_t)n;
  return buf;
}

safetensors_t* safetensors_read_dir(const char* dir) {
  safetensors_t* s = safetensors_malloc();
  char path[SAFETENSORS_MAX_STRING];
  size_t len;

  snprintf(path, sizeof(path), "%s/%s", dir, SAFETENSORS_FILE_CONFIG);
  char* text = read_file(path, &len, true);
  json_t j = {text, text + len, SAFETENSORS_FILE_CONFIG, 1};
  json_object(&j, config_member, s);
  free(text);

  snprintf(path, sizeof(path), "%s/%s", dir, SAFETENSORS_FILE_INDEX);
  text = read_file(path, &len, false);
  if (!text) {
    snprintf(path, sizeof(path), "%s/%s", dir, SAFETENSORS_FILE_SAFETENSORS);
    s->file[0] = strdup(path);
    s->file_count = 1;
  } else {
    json_t ji = {text, text + len, SAFETENSORS_FILE_INDEX, 1};
    index_ctx_t ic = {s, dir};
    json_object(&ji, index_member, &ic);
    free(text);
  }

  for (size_t i = 0; i < s->file_count; i++) {
    FILE* f = fopen(s->file[i], "rb");
    if (!f) ST_DIE("failed to open safetensors file");
    uint64_t hlen;
    if (fread(&hlen, 1, 8, f) != 8) {
      fclose(f);
      ST_DIE("failed to read safetensors header length");
    }
    char* h = malloc(hlen + 1);
    if (!h) ST_DIE("malloc failed for safetensors header");
    if (fread(h, 1, hlen, f) != hlen) ST_DIE("failed to read safetensors header");
    fclose(f);
    h[hlen] = 0;
    json_t jh = {h, h + hlen, s->file[i], 1};
    header_ctx_t hc = {s, i, (size_t)hlen, NULL};
    json_object(&jh, header_member, &hc);
    free(h);
  }

  if (s->head_dim == 0 && s->q_head_count) {
    s->head_dim = s->embedding_dim / s->q_head_count;
  }
  return s;
}

/* The reference driver releases its JSON scanner at exit
 * (source/strasgpt.c:30,287). This reader keeps no scanner state: nothing
 * to free. */
int json_scanner_lex_destroy(void) { return 0; }

safetensors_t* safetensors_read(struct options* options) {
  if (!options) ST_DIE("NULL options");
  return safetensors_read_dir(((struct options_prefix*)options)->model_dir);
}

safetensors_type_t safetensors_type_from_string(const char* s) {
  if (!s) ST_DIE("NULL string for safetensors_type_from_string");
  for (size_t i = 0; i < sizeof(safetensors_type_str) / sizeof(*safetensors_type_str); i++) {
    if (strcmp(s, safetensors_type_str[i]) == 0) return (safetensors_type_t)i;
  }
  ST_DIE("unknown data type");
  return SAFETENSORS_TYPE_F16;
}

void safetensors_file_lookup(safetensors_t* s, char* path, char* file) {
  char full[SAFETENSORS_MAX_STRING];
  snprintf(full, sizeof(full), "%s/%s", path, file);
  for (size_t i = 0; i < s->file_count; i++) {
    if (strcmp(s->file[i], full) == 0) return;
  }
  if (s->file_count >= SAFETENSORS_MAX_FILE_COUNT) ST_DIE("too many safetensors files");
  s->file[s->file_count++] = strdup(full);
}

size_t safetensors_sizeof(safetensors_type_t type) {
  switch (type) {
    case SAFETENSORS_TYPE_F16:
    case SAFETENSORS_TYPE_BF16: return 2;
    case SAFETENSORS_TYPE_F32: return 4;
    case SAFETENSORS_TYPE_U8: return 1;
  }
  ST_DIE("unknown safetensors type");
  return 0;
}

bool safetensors_aliased_out_weight(const safetensors_t* s) {
  for (size_t i = 0; i < s->tensor_count; i++) {
    if (strcmp(s->tensor[i].name, SAFETENSORS_PATTERN_OUT_WEIGHT) == 0) return false;
  }
  return true;
}

/* ------------------------------------------------------------------------ */
/* Text summaries                                                            */

static void print_config(FILE* f, const safetensors_t* s) {
  fprintf(f, "--- model_type:       %s\n", s->model_type ? s->model_type : "(null)");
  fprintf(f, "--- embedding_dim:    %zu\n", s->embedding_dim);
  fprintf(f, "--- head_dim:         %zu\n", s->head_dim);
  fprintf(f, "--- hidden_dim:       %zu\n", s->hidden_dim);
  fprintf(f, "--- layer_count:      %zu\n", s->layer_count);
  fprintf(f, "--- q_head_count:     %zu\n", s->q_head_count);
  fprintf(f, "--- kv_head_count:    %zu\n", s->kv_head_count);
  fprintf(f, "--- vocabulary_len:   %zu\n", s->vocabulary_len);
  fprintf(f, "--- context_len:      %zu\n", s->context_len);
  fprintf(f, "--- epsilon:          %g\n", s->epsilon);
  fprintf(f, "--- rope_theta:       %.1f\n", s->rope_theta);
  fprintf(f, "--- rope_interleaved: %s\n", s->rope_interleaved ? "true" : "false");
  fprintf(f, "--- mrope_sections:   ");
  if (!s->mrope_section_count) fprintf(f, "none\n");
  for (size_t i = 0; i < s->mrope_section_count; i++)
    fprintf(f, "%s%zu%s", i ? ", " : "[", s->mrope_section[i],
            i + 1 == s->mrope_section_count ? "]\n" : "");
  fprintf(f, "--- bos_token_id:     %d\n", s->bos_token_id);
  fprintf(f, "--- eos_token_id:     %d\n", s->eos_token_id);
  if (s->expert_count)
    fprintf(f, "--- experts:          %zu (top-%zu)\n", s->expert_count, s->expert_used_count);
}

void safetensors_print(FILE* f, const safetensors_t* s) {
  if (!s) {
    fprintf(f, "safetensors: NULL\n");
    return;
  }
  fprintf(f, "Safetensors:\n- Configuration:\n");
  print_config(f, s);
  fprintf(f, "- Files (%zu):\n", s->file_count);
  for (size_t i = 0; i < s->file_count; i++) fprintf(f, "--- File[%zu]: %s\n", i, s->file[i]);
  fprintf(f, "- Tensors (%zu):\n", s->tensor_count);
  for (size_t i = 0; i < s->tensor_count; i++) {
    const safetensors_tensor_t* t = &s->tensor[i];
    fprintf(f, "--- Tensor[%zu]: name=%s type=%s dim=[", i, t->name,
            safetensors_type_str[t->type]);
    for (size_t k = 0; k < t->dim_count; k++) fprintf(f, "%s%zu", k ? ", " : "", t->dim[k]);
    fprintf(f, "] size=%zu file=%zu offset=%zu\n", t->size, t->file, t->offset);
  }
}

void safetensors_print_model_infos(FILE* f, const safetensors_t* s) {
  if (!s) {
    fprintf(f, "model: NULL\n");
    return;
  }
  double total = 0, gb = 1024.0 * 1024.0 * 1024.0;
  for (size_t i = 0; i < s->tensor_count; i++) total += (double)s->tensor[i].size;
  fprintf(f, "Model:\n- Configuration:\n");
  print_config(f, s);
  fprintf(f, "- Tensors: %zu, total %.2f GB, output weight %s\n", s->tensor_count,
          total / gb, safetensors_aliased_out_weight(s) ? "aliased to embedding" : "present");
}
