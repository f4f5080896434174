/*
 * ORACLE — test infrastructure, not part of the product.
 *
 * Drives the StrasGPT reference C sources (source/transformer.c,
 * safetensors.c, sampler.c, options.c, util.c, compiled from where they lie
 * by oracle/Makefile into oracle/_ref/) on a synthetic model. The
 * reference's lex/yacc JSON front-end cannot be generated in this image,
 * so the harness fills the reference's safetensors_t itself from a plain
 * text manifest (written by tests/golden/make_golden.py from config.json
 * and the safetensors header), then runs the reference driver's greedy
 * loop (source/strasgpt.c:206-252 with --temp 0): transformer_predict over
 * the prompt inside an OpenMP team, sampler_sample, then step_count - 1
 * single-token steps.
 *
 * Manifest (whitespace separated):
 *   embedding_dim head_dim hidden_dim layer_count q_heads kv_heads vocab
 *   context_len epsilon rope_theta rope_interleaved
 *   file_count  <path>...
 *   tensor_count  (<name> <file> <offset> <size>)...
 *   token_count <ids>...   step_count
 * Output (binary, little endian): int32 generated[step_count],
 *   float32 logits_after_prompt[vocab], float32 final_norm[T][embedding_dim]
 *   for the last chunk of the prompt (the reference's state->embedding).
 * With a 4th argument L (> 0), only layers < L are loaded and run
 * (per-layer hidden-state pins).
 * Timing: stderr gets one line "timing <prefill_s> <decode_s> <decode_count>"
 * with the reference driver's boundaries (source/strasgpt.c:206-274): the
 * first transformer_predict over the prompt, and the sum of the
 * single-token steps (sampling excluded), on a monotonic clock.
 */
#include <omp.h>
#include <stdio.h>
#include <time.h>
#include <stdlib.h>
#include <string.h>

#include "options.h"
#include "safetensors.h"
#include "sampler.h"
#include "transformer.h"

static double now_s(void) {
  struct timespec ts;
  clock_gettime(CLOCK_MONOTONIC, &ts);
  return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

static int layer_of(const char* name) {
  const char* p = strstr(name, "layers.");
  if (!p) return -1;
  return atoi(p + 7);
}

int main(int argc, char** argv) {
  if (argc < 4) {
    fprintf(stderr, "usage: %s manifest out threads [layers]\n", argv[0]);
    return 2;
  }
  FILE* mf = fopen(argv[1], "r");
  if (!mf) return 2;
  int threads = atoi(argv[3]);
  long keep_layers = argc > 4 && atol(argv[4]) > 0 ? atol(argv[4]) : -1;

  safetensors_t* s = safetensors_malloc();
  int inter;
  if (fscanf(mf, "%zu %zu %zu %zu %zu %zu %zu %zu %f %f %d", &s->embedding_dim,
             &s->head_dim, &s->hidden_dim, &s->layer_count, &s->q_head_count,
             &s->kv_head_count, &s->vocabulary_len, &s->context_len, &s->epsilon,
             &s->rope_theta, &inter) != 11)
    return 3;
  s->rope_interleaved = inter != 0;
  s->eos_token_id = -1;
  if (fscanf(mf, "%zu", &s->file_count) != 1) return 3;
  for (size_t i = 0; i < s->file_count; i++) {
    char path[4096];
    if (fscanf(mf, "%4095s", path) != 1) return 3;
    s->file[i] = strdup(path);
  }
  size_t n;
  if (fscanf(mf, "%zu", &n) != 1) return 3;
  for (size_t i = 0; i < n; i++) {
    char name[1024];
    size_t file, offset, size;
    if (fscanf(mf, "%1023s %zu %zu %zu", name, &file, &offset, &size) != 4) return 3;
    if (keep_layers >= 0 && layer_of(name) >= keep_layers) continue;
    safetensors_tensor_t* t = &s->tensor[s->tensor_count++];
    t->name = strdup(name);
    t->type = SAFETENSORS_TYPE_BF16;
    t->file = file;
    t->offset = offset;
    t->size = size;
  }
  if (keep_layers >= 0) s->layer_count = (size_t)keep_layers;
  size_t T, steps;
  if (fscanf(mf, "%zu", &T) != 1) return 3;
  int* tok = malloc(T * sizeof(int));
  for (size_t i = 0; i < T; i++)
    if (fscanf(mf, "%d", &tok[i]) != 1) return 3;
  if (fscanf(mf, "%zu", &steps) != 1) return 3;
  fclose(mf);

  options_t* o = options_malloc();
  o->temperature = 0.0f;
  o->seed = 1;
  omp_set_num_threads(threads);
  transformer_t* tr = transformer_from_safetensors(s);
  sampler_t* sm = sampler_build(o, tr);
  size_t V = 0;
  float* logits = transformer_logits_malloc(tr, 1, &V);
  float* first = malloc(V * sizeof(float));
  size_t d = tr->config->embedding_dim;
  size_t last_chunk = T % TRANSFORMER_CHUNK_MAX_LEN ? T % TRANSFORMER_CHUNK_MAX_LEN
                                                    : TRANSFORMER_CHUNK_MAX_LEN;
  float* hidden = malloc(last_chunk * d * sizeof(float));
  int* gen = calloc(steps ? steps : 1, sizeof(int));
  size_t count = 0;
  int next = 0;
  double start = now_s(), prefill_s = 0.0, decode_s = 0.0;

  #pragma omp parallel
  {
    transformer_predict(tr, T, tok, 1, logits);
    #pragma omp single
    {
      prefill_s = now_s() - start;
      memcpy(first, logits, V * sizeof(float));
      memcpy(hidden, tr->state->embedding, last_chunk * d * sizeof(float));
      next = (int)sampler_sample(sm, logits, tok[T - 1]);
      gen[count++] = next;
      start = now_s();
    }
    while (count < steps) {
      transformer_predict(tr, 1, &next, 1, logits);
      #pragma omp single
      {
        decode_s += now_s() - start;
        next = (int)sampler_sample(sm, logits, next);
        gen[count++] = next;
        start = now_s();
      }
    }
  }
  fprintf(stderr, "timing %.9f %.9f %zu\n", prefill_s, decode_s, count - 1);

  FILE* out = fopen(argv[2], "wb");
  if (!out) return 4;
  fwrite(gen, sizeof(int), steps, out);
  fwrite(first, sizeof(float), V, out);
  fwrite(hidden, sizeof(float), last_chunk * d, out);
  fclose(out);
  return 0;
}
