/*
 * Error convention shared by the host code. Like the reference
 * (include/util.h:9-26), every failure prints one line prefixed with
 * "[StrasGPT] Error" and terminates the process with EXIT_FAILURE: the C
 * API has no return codes.
 */
#ifndef STRASGPT_COMMON_H
#define STRASGPT_COMMON_H

#include <stdio.h>
#include <stdlib.h>

#define ST_DIE(msg)                                                          \
  do {                                                                       \
    fprintf(stderr, "[StrasGPT] Error at %s:%d (%s): %s\n", __FILE__,        \
            __LINE__, __func__, (msg));                                      \
    exit(EXIT_FAILURE);                                                      \
  } while (0)

#define ST_ERROR(msg)                                                        \
  do {                                                                       \
    fprintf(stderr, "[StrasGPT] Error: %s\n", (msg));                        \
    exit(EXIT_FAILURE);                                                      \
  } while (0)

/* Leading fields of the reference driver's options_t (reference
 * include/options.h:18-23): the readers taking the driver's options only
 * need model_dir. */
#include <stdbool.h>
struct options_prefix {
  bool use_prompt_file;
  char* prompt_file;
  char* prompt_string;
  bool pre_tokenized;
  char* model_dir;
};

/* tokenizer.json reader of the JSON front-end (safetensors.c): appends the
 * model.vocab entries of `path` to t; dies if the file is missing or
 * malformed. */
struct tokenizer;
void st_read_tokenizer_json(const char* path, struct tokenizer* t);

#endif
