// Host-side helpers for the C-ABI entry points: argument checks, error codes and the last-error message.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/mxfp8_mlp.h"

namespace mxabi {

void set_error(const char* fmt, ...);

}  // namespace mxabi

#define MX_CHECK_ARG(cond, ...)                 \
  do {                                          \
    if (!(cond)) {                              \
      mxabi::set_error(__VA_ARGS__);            \
      return MXFP8_ERR_ARG;                     \
    }                                           \
  } while (0)

#define MX_CHECK_LAUNCH(what)                                                          \
  do {                                                                                 \
    hipError_t e_ = hipGetLastError();                                                 \
    if (e_ != hipSuccess) {                                                            \
      mxabi::set_error("%s: launch failed: %s", what, hipGetErrorString(e_));          \
      return (int)e_;                                                                  \
    }                                                                                  \
  } while (0)

static inline bool mx_aligned(const void* p, uintptr_t a) { return ((uintptr_t)p % a) == 0; }
