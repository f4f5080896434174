/*
 * ORACLE — test infrastructure, not part of the product.
 *
 * Drives the StrasGPT reference tokenizer (source/tokenizer.c and
 * source/util.c, compiled from where they lie by oracle/Makefile into
 * oracle/_ref/ref_tokenizer). The reference's tokenizer_read starts with
 * its lex/yacc parser, which this image cannot generate, so the harness
 * builds the reference's tokenizer_t from a manifest holding the
 * vocabulary keys as written in tokenizer.json and their scores, and
 * restates the steps tokenizer_read takes after parsing
 * (source/tokenizer.c:124-153): each string's byte-level map undone in
 * place (source/tokenizer.c:87-115: a two-byte UTF-8 sequence whose code
 * point is in U+0100..U+01FF becomes the byte code point - 0x100), the
 * index sorted by strcmp with qsort, the 256 one-byte strings and the
 * longest length. Everything after that is the reference's own code:
 * tokenizer_tokenize, tokenizer_decode, tokenizer_print,
 * tokenizer_print_tokens.
 *
 * Manifest (whitespace separated; byte strings in hex, "-" when empty):
 *   count (key score_hexfloat)...  bos eos
 *   text_count (bos_flag eos_flag text)...
 *   decode_count id...
 *   print_count (n id...)...
 * Output (argv[2]), one line each:
 *   per vocabulary entry, the string after the byte map is undone;
 *   per text, "n id...";
 *   per decoded id, the string's bytes.
 * argv[3] receives tokenizer_print, then tokenizer_print_tokens (4 samples)
 * of each print list. The elision line tokenizer_print writes to stderr
 * goes to the harness's stderr.
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "tokenizer.h"

static char* read_hex(FILE* f) {
  char word[1 << 16];
  if (fscanf(f, "%65535s", word) != 1) exit(3);
  if (!strcmp(word, "-")) return strdup("");
  size_t n = strlen(word) / 2;
  char* s = malloc(n + 1);
  for (size_t i = 0; i < n; i++) {
    unsigned v;
    if (sscanf(word + 2 * i, "%2x", &v) != 1) exit(3);
    s[i] = (char)v;
  }
  s[n] = 0;
  return s;
}

static void write_hex(FILE* f, const char* s) {
  if (!*s) fputc('-', f);
  for (; *s; s++) fprintf(f, "%02x", (unsigned char)*s);
  fputc('\n', f);
}

/* tokenizer_read's byte-level unmapping, restated */
static void unmap(char* str) {
  size_t r = 0, w = 0, len = strlen(str);
  while (r < len) {
    unsigned char c = (unsigned char)str[r];
    if (c >= 0xC0 && c <= 0xDF && r + 1 < len) {
      unsigned char c2 = (unsigned char)str[r + 1];
      int cp = ((c & 0x1F) << 6) | (c2 & 0x3F);
      if (cp >= 0x100 && cp <= 0x1FF) {
        str[w++] = (char)(cp - 0x100);
        r += 2;
        continue;
      }
    }
    str[w++] = str[r++];
  }
  str[w] = 0;
}

static int by_string(const void* a, const void* b) {
  return strcmp(((const tokenizer_index_t*)a)->token_string,
                ((const tokenizer_index_t*)b)->token_string);
}

int main(int argc, char** argv) {
  if (argc < 4) {
    fprintf(stderr, "usage: %s manifest out print_out\n", argv[0]);
    return 2;
  }
  FILE* mf = fopen(argv[1], "r");
  FILE* out = fopen(argv[2], "w");
  FILE* pout = fopen(argv[3], "w");
  if (!mf || !out || !pout) return 2;
  tokenizer_t* t = tokenizer_malloc();
  size_t n;
  if (fscanf(mf, "%zu", &n) != 1 || n > TOKENIZER_MAX_TOKEN_STRING) return 3;
  for (size_t i = 0; i < n; i++) {
    t->token_string[i] = read_hex(mf);
    if (fscanf(mf, "%a", &t->score[i]) != 1) return 3;
  }
  t->token_string_count = n;
  if (fscanf(mf, "%d %d", &t->bos_token_id, &t->eos_token_id) != 2) return 3;
  size_t longest = 0;
  for (size_t i = 0; i < n; i++) {
    unmap(t->token_string[i]);
    write_hex(out, t->token_string[i]);
    t->sorted_token_string[i].token_string = t->token_string[i];
    t->sorted_token_string[i].id = (int)i;
    size_t len = strlen(t->token_string[i]);
    if (len > longest) longest = len;
  }
  qsort(t->sorted_token_string, n, sizeof(tokenizer_index_t), by_string);
  for (int b = 0; b < TOKENIZER_MAX_BYTE_STRING / 2; b++) {
    t->byte_string[2 * b] = (unsigned char)b;
    t->byte_string[2 * b + 1] = 0;
  }
  t->max_token_string_len = longest;

  size_t texts;
  if (fscanf(mf, "%zu", &texts) != 1) return 3;
  for (size_t i = 0; i < texts; i++) {
    int bos, eos;
    if (fscanf(mf, "%d %d", &bos, &eos) != 2) return 3;
    char* text = read_hex(mf);
    size_t count = 0;
    int* tok = NULL;
    tokenizer_tokenize(t, text, bos != 0, eos != 0, &count, &tok);
    fprintf(out, "%zu", count);
    for (size_t k = 0; k < count; k++) fprintf(out, " %d", tok[k]);
    fputc('\n', out);
    free(tok);
    free(text);
  }
  size_t decodes;
  if (fscanf(mf, "%zu", &decodes) != 1) return 3;
  for (size_t i = 0; i < decodes; i++) {
    int id;
    if (fscanf(mf, "%d", &id) != 1) return 3;
    write_hex(out, tokenizer_decode(t, id));
  }
  tokenizer_print(pout, t);
  size_t prints;
  if (fscanf(mf, "%zu", &prints) != 1) return 3;
  for (size_t i = 0; i < prints; i++) {
    size_t m;
    if (fscanf(mf, "%zu", &m) != 1) return 3;
    int* ids = malloc((m ? m : 1) * sizeof(int));
    for (size_t k = 0; k < m; k++)
      if (fscanf(mf, "%d", &ids[k]) != 1) return 3;
    tokenizer_print_tokens(t, pout, m, ids, 4);
    free(ids);
  }
  fclose(mf);
  fclose(out);
  fclose(pout);
  tokenizer_free(t);
  return 0;
}
