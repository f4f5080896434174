/*
 * Byte-level BPE tokenizer (include/tokenizer.h), host code of the strasgpt
 * driver. Reproduces the reference tokenizer (source/tokenizer.c) id for id
 * and string for string, with its own data structures:
 *  - reading (reference :120-156): model.vocab of tokenizer.json in file
 *    order (ids are positions, scores the numbers the file gives); in each
 *    string, a two-byte UTF-8 sequence whose code point falls in
 *    U+0100..U+01FF (lead byte 0xC4..0xC7, the next byte's continuation
 *    bits not checked) becomes the byte code point - 0x100, everything else
 *    is kept as written; an index sorted by strcmp with equal strings in id
 *    order (what glibc's merge-sort qsort gives the reference); 256
 *    one-byte strings; the longest string length;
 *  - lookup: bisection over that index with the midpoint (l + u) / 2, so
 *    that among equal strings the id found is the one glibc's bsearch
 *    finds;
 *  - encoding (reference :225-398): a code point is a byte plus up to three
 *    following continuation bytes; its id, or one id per byte (value + 3)
 *    when the vocabulary lacks it; then, while a merge exists, the adjacent
 *    pair whose concatenation has the highest score (the leftmost on equal
 *    scores; scores must exceed -1e10) is replaced by that token, or, when
 *    no pair merges, the best triple. The reference rebuilds and looks up
 *    every pair string on each merge; here the merge result of each
 *    position's pair and triple is cached in a doubly linked token list and
 *    recomputed only next to a merge, so a merge costs one scan of cached
 *    scores and at most five lookups. An id without a vocabulary string (a
 *    BOS id among the added tokens, a byte id past a small vocabulary)
 *    concatenates as "(null)", the text glibc prints for the null string
 *    the reference passes in that case.
 */
#define _GNU_SOURCE
#include "tokenizer.h"

#include <ctype.h>
#include <float.h>
#include <string.h>

#include "common.h"

tokenizer_t* tokenizer_malloc(void) {
  tokenizer_t* t = calloc(1, sizeof(tokenizer_t));
  if (!t) ST_DIE("failed to malloc for tokenizer_t");
  return t;
}

void tokenizer_free(tokenizer_t* t) {
  if (!t) return;
  for (size_t i = 0; i < t->token_string_count; i++) free(t->token_string[i]);
  free(t);
}

static void print_entry(FILE* f, const tokenizer_t* t, size_t i) {
  fprintf(f, "--- Token string[%6zu]: score=%10.3f string=%s\n", i, t->score[i],
          t->token_string[i]);
}

void tokenizer_print(FILE* f, const tokenizer_t* t) {
  if (!t) {
    fprintf(f, "Tokenizer: NULL\n");
    return;
  }
  const size_t n = t->token_string_count, k = TOKENIZER_MAX_PRINT;
  fprintf(f, "Tokenizer:\n- Special tokens:\n");
  fprintf(f, "--- bos_token_id: %d\n--- eos_token_id: %d\n", t->bos_token_id, t->eos_token_id);
  fprintf(f, "- Token strings (%zu):\n", n);
  const size_t head = n < k ? n : k;
  for (size_t i = 0; i < head; i++) print_entry(f, t, i);
  /* the reference writes this elision line to stderr whatever f is */
  if (2 * k < n) fprintf(stderr, "--- ...\n");
  for (size_t i = 2 * k < n ? n - k : head; i < n; i++) print_entry(f, t, i);
  fprintf(f, "- Max token string length: %zu\n", t->max_token_string_len);
}

/* Undoes the byte-to-character map of byte-level BPE in place: lead byte
 * 0xC4..0xC7 followed by any byte b2 is the byte ((lead & 3) << 6) |
 * (b2 & 0x3F). */
static void unmap_bytes(char* s) {
  const size_t n = strlen(s);
  size_t w = 0;
  for (size_t r = 0; r < n; w++) {
    const unsigned char b = (unsigned char)s[r];
    if (b >= 0xC4 && b <= 0xC7 && r + 1 < n) {
      s[w] = (char)(((b & 3u) << 6) | ((unsigned char)s[r + 1] & 0x3Fu));
      r += 2;
    } else {
      s[w] = s[r++];
    }
  }
  s[w] = 0;
}

static int by_string_then_id(const void* a, const void* b) {
  const tokenizer_index_t* x = a;
  const tokenizer_index_t* y = b;
  const int c = strcmp(x->token_string, y->token_string);
  return c ? c : (x->id > y->id) - (x->id < y->id);
}

tokenizer_t* tokenizer_read_dir(const char* dir) {
  if (!dir) ST_DIE("NULL model directory");
  char path[4096];
  snprintf(path, sizeof(path), "%s/%s", dir, TOKENIZER_FILE);
  tokenizer_t* t = tokenizer_malloc();
  st_read_tokenizer_json(path, t);
  const size_t n = t->token_string_count;
  size_t longest = 0;
  for (size_t i = 0; i < n; i++) {
    unmap_bytes(t->token_string[i]);
    const size_t len = strlen(t->token_string[i]);
    if (len > longest) longest = len;
    t->sorted_token_string[i].token_string = t->token_string[i];
    t->sorted_token_string[i].id = (int)i;
  }
  qsort(t->sorted_token_string, n, sizeof(tokenizer_index_t), by_string_then_id);
  for (int b = 0; b < TOKENIZER_MAX_BYTE_STRING / 2; b++) {
    t->byte_string[2 * b] = (unsigned char)b;
    t->byte_string[2 * b + 1] = 0;
  }
  t->max_token_string_len = longest;
  return t;
}

tokenizer_t* tokenizer_read(struct options* options) {
  if (!options) ST_DIE("NULL options");
  return tokenizer_read_dir(((struct options_prefix*)options)->model_dir);
}

void tokenizer_print_token_string(FILE* f, char* s) {
  if (!s || !s[0]) return;
  if (!s[1] && !(isprint((unsigned char)s[0]) || isspace((unsigned char)s[0]))) return;
  fprintf(f, "%s", s);
  fflush(f);
}

char* tokenizer_decode(tokenizer_t* t, int token) {
  if (token == t->bos_token_id) return (char*)TOKENIZER_STRING_TOKEN_BOS;
  if (token == t->eos_token_id) return (char*)TOKENIZER_STRING_TOKEN_EOS;
  if (token < 0 || (size_t)token >= t->token_string_count) return (char*)"<|unknown_token|>";
  char* s = t->token_string[token];
  unsigned char byte;
  /* raw-byte entries such as "<0x0A>" (same conversion rules as the
   * reference: sscanf's %X, at most two characters) */
  if (sscanf(s, "<0x%02hhX>", &byte) == 1) s = (char*)t->byte_string + 2 * byte;
  return s;
}

/* Id of the vocabulary entry equal to key, -1 if none. */
static int find_id(const tokenizer_t* t, const char* key) {
  size_t lo = 0, hi = t->token_string_count;
  while (lo < hi) {
    const size_t mid = (lo + hi) / 2;
    const int c = strcmp(key, t->sorted_token_string[mid].token_string);
    if (c < 0) hi = mid;
    else if (c > 0) lo = mid + 1;
    else return t->sorted_token_string[mid].id;
  }
  return -1;
}

static const char* text_of(const tokenizer_t* t, int id) {
  if (id < 0 || (size_t)id >= t->token_string_count || !t->token_string[id]) return "(null)";
  return t->token_string[id];
}

typedef struct {
  const tokenizer_t* t;
  int* id;            /* token per node */
  int* prev;          /* linked list over nodes, -1 at the ends */
  int* next;
  int* pair;          /* merge result of (node, next), -1 if none */
  int* triple;        /* merge result of (node, next, next of next) */
  char* buf;          /* concatenation buffer */
  size_t cap;
} merger_t;

static int merged_id(merger_t* m, int a, int b, int c) {
  const char* s[3] = {text_of(m->t, a), text_of(m->t, b), c >= 0 ? text_of(m->t, c) : ""};
  size_t len[3], total = 0;
  for (int i = 0; i < 3; i++) total += len[i] = strlen(s[i]);
  /* longer than every vocabulary string: no entry can match */
  if (total > m->t->max_token_string_len) return -1;
  char* p = m->buf;
  for (int i = 0; i < 3; i++) {
    memcpy(p, s[i], len[i]);
    p += len[i];
  }
  *p = 0;
  return find_id(m->t, m->buf);
}

static void refresh(merger_t* m, int node) {
  if (node < 0) return;
  const int n1 = m->next[node];
  const int n2 = n1 >= 0 ? m->next[n1] : -1;
  m->pair[node] = n1 >= 0 ? merged_id(m, m->id[node], m->id[n1], -1) : -1;
  m->triple[node] = n2 >= 0 ? merged_id(m, m->id[node], m->id[n1], m->id[n2]) : -1;
}

/* Leftmost node whose cached merge (pair or triple table) scores highest
 * above -1e10; -1 if none. */
static int best_node(const merger_t* m, const int* table, int head) {
  float best = -1e10f;
  int where = -1;
  for (int i = head; i >= 0; i = m->next[i]) {
    const int id = table[i];
    if (id != -1 && m->t->score[id] > best) {
      best = m->t->score[id];
      where = i;
    }
  }
  return where;
}

void tokenizer_tokenize(tokenizer_t* t, char* text, bool bos, bool eos, size_t* token_count,
                        int** token_out) {
  if (!text) ST_DIE("cannot encode NULL text");
  const size_t text_len = strlen(text);
  int* tok = malloc((text_len + 3) * sizeof(int));
  if (!tok) ST_DIE("failed to malloc for tokens");
  *token_out = tok;
  size_t n = 0;
  if (bos) tok[n++] = t->bos_token_id;

  /* code points: a byte and up to three following continuation bytes */
  char cp[5];
  for (size_t i = 0; i < text_len;) {
    size_t len = 0;
    cp[len++] = text[i++];
    while (len < 4 && i < text_len && ((unsigned char)text[i] & 0xC0) == 0x80) cp[len++] = text[i++];
    cp[len] = 0;
    const int id = find_id(t, cp);
    if (id != -1) {
      tok[n++] = id;
    } else {
      for (size_t k = 0; k < len; k++) tok[n++] = (unsigned char)cp[k] + 3;
    }
  }

  if (n > 1) {
    merger_t m;
    m.t = t;
    m.cap = 3 * t->max_token_string_len + 3 * 8 + 1;
    m.buf = malloc(m.cap);
    int* mem = malloc(5 * n * sizeof(int));
    if (!m.buf || !mem) ST_DIE("failed to malloc for token merges");
    m.id = mem;
    m.prev = mem + n;
    m.next = mem + 2 * n;
    m.pair = mem + 3 * n;
    m.triple = mem + 4 * n;
    for (size_t i = 0; i < n; i++) {
      m.id[i] = tok[i];
      m.prev[i] = (int)i - 1;
      m.next[i] = i + 1 < n ? (int)i + 1 : -1;
    }
    for (size_t i = 0; i < n; i++) refresh(&m, (int)i);
    const int head = 0; /* node 0 is never removed: merges keep the left node */
    for (;;) {
      int at = best_node(&m, m.pair, head);
      int width = 2;
      if (at < 0) {
        at = best_node(&m, m.triple, head);
        width = 3;
      }
      if (at < 0) break;
      m.id[at] = width == 2 ? m.pair[at] : m.triple[at];
      for (int k = 1; k < width; k++) {
        const int gone = m.next[at];
        m.next[at] = m.next[gone];
        if (m.next[gone] >= 0) m.prev[m.next[gone]] = at;
      }
      const int p1 = m.prev[at];
      refresh(&m, at);
      refresh(&m, p1);
      if (p1 >= 0) refresh(&m, m.prev[p1]);
    }
    n = 0;
    for (int i = head; i >= 0; i = m.next[i]) tok[n++] = m.id[i];
    free(mem);
    free(m.buf);
  }

  if (eos) tok[n++] = t->eos_token_id;
  *token_count = n;
}

static void print_token_line(tokenizer_t* t, FILE* f, size_t i, int id) {
  fprintf(f, "- Token[%4zu]: %6d (\"", i, id);
  tokenizer_print_token_string(f, tokenizer_decode(t, id));
  fprintf(f, "\")\n");
}

void tokenizer_print_tokens(tokenizer_t* t, FILE* f, size_t count, int* token, size_t sample) {
  fprintf(f, "Tokens (%zu):\n", count);
  const size_t head = count < sample ? count : sample;
  for (size_t i = 0; i < head; i++) print_token_line(t, f, i, token[i]);
  if (2 * sample < count) fprintf(f, "- ...\n");
  for (size_t i = 2 * sample < count ? count - sample : head; i < count; i++)
    print_token_line(t, f, i, token[i]);
  fflush(f);
}
