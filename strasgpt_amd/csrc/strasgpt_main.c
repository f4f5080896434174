/*
 * strasgpt: generation driver over libstrasgpt_hip with the reference
 * driver's flags and output (reference source/options.c:102-224,
 * source/strasgpt.c:100-281):
 *   -m <dir>  -n <steps>  -t <threads>  -s <seed>  --temp <t>  --top-k <k>
 *   --top-p <p>  --presence-penalty <x>  -p <prompt> | -f <file>
 *   --pre-tokenized (the prompt is space/comma separated ids, no BOS
 *   added; otherwise the text is tokenized with tokenizer.json and BOS is
 *   prepended)
 * plus:
 *   --host-loop   run the reference loop literally (source/strasgpt.c:
 *                 206-252): transformer_predict from every thread of an
 *                 OpenMP team, logits to the host, the token chosen by the
 *                 device argmax (--temp 0) or the device sampler;
 *   --ids         print the generated ids on one line instead of their
 *                 strings;
 *   --show-model  print the model summary and exit;
 *   --show-safetensors  print the safetensors summary and exit;
 *   --instruct    wrap the prompt ids in the model family's chat template
 *                 (no BOS added to a text prompt; source/strasgpt.c:
 *                 170-179).
 * Default: transformer_generate_greedy / transformer_generate_sampled
 * (device-resident decode loop). Generated token strings go to stdout as
 * in the reference (the first token always, then up to EOS, printed as
 * <|end_of_text|>); the tokenizer summary, the prompt tokens and the timing
 * lines go to stderr with the reference's boundaries: prefill = first
 * predict over the prompt, decode = sum of the single-token steps
 * (source/strasgpt.c:206-274). --presence-penalty is range-checked and,
 * as in the reference (whose sampler_build never reads it), not applied.
 */
#define _GNU_SOURCE
#include <omp.h>
#include <stdbool.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <sys/resource.h>
#include <time.h>

#include "safetensors.h"
#include "sampler_hip.h"
#include "tokenizer.h"
#include "transformer.h"
#include "transformer_hip.h"

static double now_s(void) {
  struct timespec ts;
  clock_gettime(CLOCK_MONOTONIC, &ts);
  return ts.tv_sec + 1e-9 * ts.tv_nsec;
}

/* --instruct: ids put before and after the prompt per model family,
 * chosen by a substring of config.json's model_type, first match wins; no
 * match leaves the prompt as it is. The ids and the order of the checks are
 * the reference's (source/util.c:514-575). */
typedef struct {
  const char* match[2];
  int before[20];
  int n_before;
  int after[8];
  int n_after;
} chat_template_t;

static const chat_template_t kChatTemplates[] = {
    {{"qwen3", "qwen3_vl"},
     {151644, 8948, 198, 2610, 525, 264, 10950, 17847, 624, 151645, 198, 151644, 872, 198},
     14,
     {198, 151645, 198, 151644, 77091},
     5},
    {{"Mistral", "mistral"}, {1, 1, 3}, 3, {4}, 1},
    {{"Llama", "llama"},
     {128000, 128000, 198, 128006, 9125, 128007, 198, 2675, 527, 264, 11190, 18328, 627, 128009, 198,
      128006, 882, 128007, 198},
     19,
     {198, 128009, 198, 128006, 78191, 128007},
     6},
};

static int* wrap_instruct(int* tok, size_t* n, const char* model_type) {
  if (!model_type) return tok;
  for (size_t t = 0; t < sizeof kChatTemplates / sizeof kChatTemplates[0]; t++) {
    const chat_template_t* c = &kChatTemplates[t];
    if (!strstr(model_type, c->match[0]) && !strstr(model_type, c->match[1])) continue;
    int* out = malloc((c->n_before + *n + c->n_after) * sizeof(int));
    if (!out) {
      fprintf(stderr, "[StrasGPT] Error: out of memory for the instruction tokens\n");
      exit(EXIT_FAILURE);
    }
    memcpy(out, c->before, c->n_before * sizeof(int));
    memcpy(out + c->n_before, tok, *n * sizeof(int));
    memcpy(out + c->n_before + *n, c->after, c->n_after * sizeof(int));
    free(tok);
    *n += c->n_before + c->n_after;
    return out;
  }
  return tok;
}

static void usage(const char* argv0, int status) {
  fprintf(stderr,
          "Usage: %s -m <model_dir> [-n steps] [-t threads] [-s seed] [--temp t] [--top-k k]\n"
          "       [--top-p p] [--presence-penalty x] (-p <prompt> | -f <file>) [--pre-tokenized]\n"
          "       [--instruct] [--host-loop] [--ids] [--show-model] [--show-safetensors]\n",
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

/* Prompt file contents, one trailing newline removed (reference
 * source/strasgpt.c:133-157). */
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
  if (!s || fread(s, 1, (size_t)n, f) != (size_t)n) {
    fprintf(stderr, "[StrasGPT] Error: can't read prompt file\n");
    exit(EXIT_FAILURE);
  }
  s[n] = 0;
  if (n > 0 && s[n - 1] == '\n') s[n - 1] = 0;
  fclose(f);
  return s;
}

static float parse_float(const char* flag, const char* v, float lo, float hi) {
  char* end;
  float x = strtof(v, &end);
  if (end == v || *end || !(x >= lo && x <= hi)) {
    fprintf(stderr, "[StrasGPT] Error: %s expects a number in [%g, %g]\n", flag, lo, hi);
    exit(EXIT_FAILURE);
  }
  return x;
}

/* One generated token to stdout as the reference prints it. Returns false
 * when it ends the generation (EOS after the first token). */
static bool emit(tokenizer_t* tk, int id, size_t index, int eos, bool ids_only) {
  if (ids_only) {
    printf("%s%d", index ? " " : "", id);
    return index == 0 || id != eos;
  }
  if (index > 0 && id == eos) {
    fputs(TOKENIZER_STRING_TOKEN_EOS, stdout);
    return false;
  }
  tokenizer_print_token_string(stdout, tokenizer_decode(tk, id));
  return true;
}

int main(int argc, char** argv) {
  const char* model = ".";
  const char* prompt = "Once upon a time";
  char* file_text = NULL;
  size_t steps = 256, top_k = 40;
  int threads = 1;
  unsigned long long seed = 0;
  float temp = 1.0f, top_p = 0.9f;
  bool pre_tokenized = false, host_loop = false, show_model = false, ids_only = false;
  bool show_safetensors = false, instruct = false;
  for (int i = 1; i < argc; i++) {
    const char* a = argv[i];
    const char* v = i + 1 < argc ? argv[i + 1] : NULL;
    if (!strcmp(a, "-h") || !strcmp(a, "--help")) usage(argv[0], EXIT_SUCCESS);
    else if (!strcmp(a, "--pre-tokenized")) pre_tokenized = true;
    else if (!strcmp(a, "--host-loop")) host_loop = true;
    else if (!strcmp(a, "--show-model")) show_model = true;
    else if (!strcmp(a, "--show-safetensors")) show_safetensors = true;
    else if (!strcmp(a, "--instruct")) instruct = true;
    else if (!strcmp(a, "--ids")) ids_only = true;
    else if (!v) usage(argv[0], EXIT_FAILURE);
    else if (!strcmp(a, "-m")) model = argv[++i];
    else if (!strcmp(a, "-n")) steps = strtoull(argv[++i], NULL, 10);
    else if (!strcmp(a, "-t")) threads = atoi(argv[++i]);
    else if (!strcmp(a, "-s")) seed = strtoull(argv[++i], NULL, 10);
    else if (!strcmp(a, "--temp")) temp = parse_float(a, argv[++i], 0.0f, 1e30f);
    else if (!strcmp(a, "--top-k")) top_k = strtoull(argv[++i], NULL, 10);
    else if (!strcmp(a, "--top-p")) top_p = parse_float(a, argv[++i], 0.0f, 1.0f);
    else if (!strcmp(a, "--presence-penalty")) (void)parse_float(a, argv[++i], 0.0f, 2.0f);
    else if (!strcmp(a, "-p")) prompt = argv[++i];
    else if (!strcmp(a, "-f")) prompt = file_text = read_text(argv[++i]);
    else usage(argv[0], EXIT_FAILURE);
  }

  if (steps == 0) steps = 1; /* the reference always predicts the first token */
  safetensors_t* st = safetensors_read_dir(model);
  if (show_safetensors) {
    safetensors_print(stderr, st);
    safetensors_free(st);
    return EXIT_SUCCESS;
  }
  if (show_model) {
    safetensors_print_model_infos(stderr, st);
    safetensors_free(st);
    return EXIT_SUCCESS;
  }
  tokenizer_t* tk = tokenizer_read_dir(model);
  tk->bos_token_id = st->bos_token_id;
  tk->eos_token_id = st->eos_token_id;
  tokenizer_print(stderr, tk);

  size_t n_tok = 0;
  int* tok = NULL;
  if (pre_tokenized) tok = parse_ids(prompt, &n_tok);
  else tokenizer_tokenize(tk, (char*)prompt, !instruct, false, &n_tok, &tok);
  if (n_tok < 1) {
    fprintf(stderr, "[StrasGPT] Error: expected at least 1 prompt token\n");
    return EXIT_FAILURE;
  }
  if (instruct) tok = wrap_instruct(tok, &n_tok, st->model_type);
  tokenizer_print_tokens(tk, stderr, n_tok, tok, 4);
  fprintf(stderr, "\n\033[1;34m");
  for (size_t i = 0; i < n_tok; i++) tokenizer_print_token_string(stderr, tokenizer_decode(tk, tok[i]));
  fprintf(stderr, "\033[0m");
  const int eos = st->eos_token_id;

  transformer_t* t = transformer_from_safetensors(st);
  transformer_print(stderr, t);
  sampler_hip_t* smp = NULL;
  if (temp != 0.0f) smp = sampler_hip_build(t->config->vocabulary_len, temp, top_k, top_p, seed);

  int* out = calloc(steps, sizeof(int));
  size_t produced = 0;
  double prefill_s = 0, decode_s = 0;
  if (!host_loop) {
    transformer_timing_t tm;
    produced = smp ? transformer_generate_sampled(t, n_tok, tok, steps, eos, smp, out, &tm)
                   : transformer_generate_greedy(t, n_tok, tok, steps, eos, out, &tm);
    prefill_s = tm.prefill_s;
    decode_s = tm.decode_s;
    for (size_t i = 0; i < produced; i++) emit(tk, out[i], i, eos, ids_only);
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
        next = smp ? (int)sampler_hip_sample(smp, logits, tok[n_tok - 1])
                   : (int)sampler_argmax(logits, V);
        out[produced] = next;
        emit(tk, next, produced++, eos, ids_only);
        start = now_s();
      }
      while (produced < steps && go) {
        transformer_predict(t, 1, &next, 1, logits);
        #pragma omp single
        {
          decode_s += now_s() - start;
          next = smp ? (int)sampler_hip_sample(smp, logits, next) : (int)sampler_argmax(logits, V);
          out[produced] = next;
          go = emit(tk, next, produced++, eos, ids_only);
          start = now_s();
        }
      }
    }
    free(logits);
  }
  printf("\n");
  // host peak resident set (Linux: ru_maxrss in KiB), as the reference reports it
  struct rusage ru;
  const double rss_gb = getrusage(RUSAGE_SELF, &ru) == 0 ? ru.ru_maxrss / (1024.0 * 1024.0) : -1.0;
  fprintf(stderr, "\nMax memory used (RSS): %.2f GB", rss_gb);
  fprintf(stderr, "\nPrompt processing (prefill): %4zu tokens in %7.3f s (%f token/s)\n", n_tok,
          prefill_s, n_tok / prefill_s);
  if (produced > 1)
    fprintf(stderr, "Token generation  (decode):  %4zu tokens in %7.3f s (%f token/s)\n",
            produced - 1, decode_s, (produced - 1) / decode_s);
  if (smp) sampler_hip_free(smp);
  transformer_free(t);
  tokenizer_free(tk);
  safetensors_free(st);
  free(out);
  free(tok);
  free(file_text);
  return EXIT_SUCCESS;
}
