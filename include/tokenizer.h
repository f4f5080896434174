/*
 * Byte-level BPE tokenizer of the strasgpt driver: vocabulary read from the
 * model directory's tokenizer.json, prompt text to token ids, token ids to
 * printable strings.
 *
 * Drop-in replacement for the reference tokenizer (include/tokenizer.h:1-56
 * and source/tokenizer.c of StrasGPT): same function names, arguments and
 * die-on-error behaviour. tokenizer_t keeps the reference's field order and
 * array sizes (include/tokenizer.h:17-33), because the reference driver
 * reads and writes bos_token_id / eos_token_id in place
 * (source/strasgpt.c:114-115) and so must see them at the same offsets.
 * tokenizer_read_dir is an addition (the model directory without the
 * driver's options struct).
 */
#ifndef TOKENIZER_H
# define TOKENIZER_H

#include <stdbool.h>
#include <stddef.h>
#include <stdio.h>

#ifdef __cplusplus
extern "C" {
#endif

struct options;

#define TOKENIZER_FILE             "tokenizer.json"
#define TOKENIZER_MAX_PRINT        4
#define TOKENIZER_MAX_TOKEN_STRING 262144 /* vocabulary entries read at most */
#define TOKENIZER_MAX_BYTE_STRING  512    /* 256 one-byte strings, each NUL-terminated */
#define TOKENIZER_STRING_TOKEN_BOS "<|begin_of_text|>"
#define TOKENIZER_STRING_TOKEN_EOS "<|end_of_text|>"

/* One entry of the vocabulary sorted by string (strcmp order; equal strings
 * keep vocabulary order). */
typedef struct {
  char* token_string;
  int id;
} tokenizer_index_t;

typedef struct tokenizer {
  size_t token_string_count;                   /* entries of model.vocab, in file order */
  char* token_string[TOKENIZER_MAX_TOKEN_STRING];  /* id -> bytes (byte-level map undone) */
  float score[TOKENIZER_MAX_TOKEN_STRING];     /* id -> the number the vocab maps it to */
  tokenizer_index_t sorted_token_string[TOKENIZER_MAX_TOKEN_STRING];
  size_t max_token_string_len;                 /* longest token string, in bytes */
  unsigned char byte_string[TOKENIZER_MAX_BYTE_STRING]; /* byte b at [2b], NUL at [2b+1] */
  int bos_token_id;
  int eos_token_id;
} tokenizer_t;

/* Zeroed tokenizer (dies if out of memory). */
tokenizer_t* tokenizer_malloc(void);
/* Frees the token strings and the struct; NULL is accepted. */
void tokenizer_free(tokenizer_t* tokenizer);
/* Special ids, the first and last TOKENIZER_MAX_PRINT token strings with
 * their scores, the longest string length. */
void tokenizer_print(FILE* f, const tokenizer_t* tokenizer);
/* Reads <options->model_dir>/tokenizer.json (reference source/tokenizer.c:
 * 120-156); dies if the file is missing or malformed. bos/eos ids are left
 * at 0 for the caller to set from the model config. */
tokenizer_t* tokenizer_read(struct options* options);
tokenizer_t* tokenizer_read_dir(const char* model_dir);

/* Prints a token string unless it is empty or a single byte that is neither
 * printable nor white space. */
void tokenizer_print_token_string(FILE* f, char* token_string);
/* String of a token id: the BOS/EOS strings for those ids,
 * "<|unknown_token|>" outside the vocabulary, the raw byte for "<0xHH>"
 * entries (reference source/tokenizer.c:181-202). */
char* tokenizer_decode(tokenizer_t* t, int token);
/* Encodes text (reference source/tokenizer.c:225-398): optional BOS, one id
 * per UTF-8 code point found in the vocabulary (else one id per byte, byte
 * value + 3), then repeated merges of the highest-scoring adjacent pair
 * whose concatenation is in the vocabulary (the leftmost on equal scores),
 * or of a triple when no pair merges; optional EOS. *token is malloc'ed
 * (strlen(text) + 3 entries); the caller frees it. */
void tokenizer_tokenize(tokenizer_t* t, char* text, bool bos, bool eos, size_t* token_count,
                        int** token);
/* "Tokens (n):" then the first and last sample_count ids with their
 * strings. */
void tokenizer_print_tokens(tokenizer_t* tokenizer, FILE* f, size_t token_count, int* token,
                            size_t sample_count);

#ifdef __cplusplus
}
#endif

#endif /* TOKENIZER_H */
