/*
 * strasgpt: greedy generation driver over libstrasgpt_hip, accepting the
 * reference driver's benchmark flags (reference source/options.c:102-224):
 *   -m <dir>  -n <steps>  -t <threads>  -s <seed>  --temp 0
 *   -p <prompt> | -f <file>  with --pre-tokenized (space/comma separated ids)
 * plus:
 *   --host-loop   run the reference loop literally (source/strasgpt.c:
 *                 206-252): transformer_predict from every thread of an
 *                 OpenMP team, logits to the host, argmax on the host;
 *   --show-model  print the model summary and exit.
 * Default: transformer_generate_greedy (device-resident decode loop).
 * Generated ids go to stdout, one line; timing lines go to stderr with the
 * reference's boundaries: prefill = first predict over the prompt, decode =
 * sum of the single-token steps (source/strasgpt.c:206-274).
 */
#define _GNU_SOURCE
#include <omp.h>
#include <stdbool.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "safetensors.h"
#include "transformer.h"
#include "transformer_hip.h"

static double now_s(void) {
  struct timespec ts;
  clock_gettime(CLOCK_MONOTONIC, &ts);
  return ts.tv_sec + 1e-9 * ts.tv_nsec;
}

static void usage(const char* argv0, int status) {
  fprintf(stderr,
          "Usage: %s -m <model_dir> [-n steps] [-t threads] [--temp 0] "
          "--pre-tokenized (-p \"ids\" | -f file) [--host-loop] [--show-model]\n",
          argv0);
  exit(status);
}

static int* parse_ids(const char* text, size_t* count) {
  size_t cap = 64, n = 0;
  int* ids = malloc(cap * sizeof(int));
  const char* p = text;
  while (*p) {
    while (*p && strchr(" \t\r\n,", *p)) p++;
    if (!*p) break;
    char* end;
    long v = strtol(p, &end, 10);
    if (end == p || (*end && !strchr(" \t\r\n,", *end))) {
      fprintf(stderr, "[StrasGPT] Error: invalid token ID near: %.20s\n", p);
      exit(EXIT_FAILURE);
    }
    if (n == cap) ids = realloc(ids, (cap *= 2) * sizeof(int));
    ids[n++] = (int)v;
    p = end;
  }
  *count = n;
  return ids;
}

static char* read_text(const char* path) {
  FILE* f = fopen(path, "rb");
  if (!f) {
    fprintf(stderr, "[StrasGPT] Error: can't open prompt file\n");
    exit(EXIT_FAILURE);
  }
  fseek(f, 0, SEEK_END);
  long n = ftell(f);
  fseek(f, 0, SEEK_SET);
  char* s = malloc((size_t)n + 1);
  if (fread(s, 1, (size_t)n, f) != (size_t)n) exit(EXIT_FAILURE);
  s[n] = 0;
  fclose(f);
  return s;
}

int main(int argc, char** argv) {
  const char* model = ".";
  const char* prompt = NULL;
  char* file_text = NULL;
  size_t steps = 256;
  int threads = 1;
  float temp = 1.0f;
  bool pre_tokenized = false, host_loop = false, show_model = false;
  for (int i = 1; i < argc; i++) {
    const char* a = argv[i];
    const char* v = i + 1 < argc ? argv[i + 1] : NULL;
    if (!strcmp(a, "-h") || !strcmp(a, "--help")) usage(argv[0], EXIT_SUCCESS);
    else if (!strcmp(a, "--pre-tokenized")) pre_tokenized = true;
    else if (!strcmp(a, "--host-loop")) host_loop = true;
    else if (!strcmp(a, "--show-model")) show_model = true;
    else if (!v) usage(argv[0], EXIT_FAILURE);
    else if (!strcmp(a, "-m")) model = argv[++i];
    else if (!strcmp(a, "-n")) steps = strtoull(argv[++i], NULL, 10);
    else if (!strcmp(a, "-t")) threads = atoi(argv[++i]);
    else if (!strcmp(a, "-s")) ++i;
    else if (!strcmp(a, "--temp")) temp = strtof(argv[++i], NULL);
    else if (!strcmp(a, "-p")) prompt = argv[++i];
    else if (!strcmp(a, "-f")) prompt = file_text = read_text(argv[++i]);
    else usage(argv[0], EXIT_FAILURE);
  }

  safetensors_t* st = safetensors_read_dir(model);
  if (show_model) {
    safetensors_print_model_infos(stderr, st);
    safetensors_free(st);
    return EXIT_SUCCESS;
  }
  if (temp != 0.0f) {
    fprintf(stderr, "[StrasGPT] Error: this driver implements greedy decoding only (--temp 0)\n");
    return EXIT_FAILURE;
  }
  if (!pre_tokenized || !prompt) {
    fprintf(stderr, "[StrasGPT] Error: pass token ids with --pre-tokenized and -p/-f\n");
    return EXIT_FAILURE;
  }
  size_t n_tok = 0;
  int* tok = parse_ids(prompt, &n_tok);
  if (n_tok < 1) {
    fprintf(stderr, "[StrasGPT] Error: expected at least 1 prompt token\n");
    return EXIT_FAILURE;
  }
  int eos = st->eos_token_id;

  transformer_t* t = transformer_from_safetensors(st);
  transformer_print(stderr, t);

  int* out = calloc(steps ? steps : 1, sizeof(int));
  size_t produced = 0;
  double prefill_s = 0, decode_s = 0;
  if (!host_loop) {
    transformer_timing_t tm;
    produced = transformer_generate_greedy(t, n_tok, tok, steps, eos, out, &tm);
    prefill_s = tm.prefill_s;
    decode_s = tm.decode_s;
  } else {
    size_t V = 0;
    float* logits = transformer_logits_malloc(t, 1, &V);
    omp_set_num_threads(threads > 0 ? threads : 1);
    double start = now_s();
    int next = 0;
    bool go = true;
    #pragma omp parallel shared(go, next, produced, start, prefill_s, decode_s)
    {
      transformer_predict(t, n_tok, tok, 1, logits);
      #pragma omp single
      {
        prefill_s = now_s() - start;
        size_t best = 0;
        for (size_t v = 1; v < V; v++)
          if (logits[v] > logits[best]) best = v;
        next = (int)best;
        out[produced++] = next;
        go = next != eos;
        start = now_s();
      }
      while (produced < steps && go) {
        transformer_predict(t, 1, &next, 1, logits);
        #pragma omp single
        {
          decode_s += now_s() - start;
          size_t best = 0;
          for (size_t v = 1; v < V; v++)
            if (logits[v] > logits[best]) best = v;
          next = (int)best;
          out[produced++] = next;
          go = next != eos;
          start = now_s();
        }
      }
    }
    free(logits);
  }
  for (size_t i = 0; i < produced; i++) printf("%s%d", i ? " " : "", out[i]);
  printf("\n");
  fprintf(stderr, "Prompt processing (prefill): %4zu tokens in %7.3f s (%f token/s)\n", n_tok,
          prefill_s, n_tok / prefill_s);
  if (produced > 1)
    fprintf(stderr, "Token generation  (decode):  %4zu tokens in %7.3f s (%f token/s)\n",
            produced - 1, decode_s, (produced - 1) / decode_s);
  transformer_free(t);
  safetensors_free(st);
  free(out);
  free(tok);
  free(file_text);
  return EXIT_SUCCESS;
}
