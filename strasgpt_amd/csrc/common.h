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

#endif
