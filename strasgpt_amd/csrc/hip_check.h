// HIP runtime errors follow the library's die-with-message convention.
#pragma once

#include <hip/hip_runtime.h>

#include "common.h"

#define HIP_CHECK(expr)                                                      \
  do {                                                                       \
    hipError_t err_ = (expr);                                                \
    if (err_ != hipSuccess) {                                                \
      char msg_[512];                                                        \
      snprintf(msg_, sizeof(msg_), "HIP error '%s' from %s",                 \
               hipGetErrorString(err_), #expr);                              \
      ST_DIE(msg_);                                                          \
    }                                                                        \
  } while (0)
