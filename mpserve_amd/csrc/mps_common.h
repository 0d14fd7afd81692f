// Shared host-side helpers of libmpserve_amd: per-thread error text and HIP checks.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <string>

#include "mpserve_amd.h"

namespace mps {

// Last error message of the calling thread (returned by mps_last_error()).
std::string &last_error();

inline int fail(int code, const char *fmt, ...) {
  char buf[1024];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  last_error() = buf;
  return code;
}

inline int hip_fail(hipError_t e, const char *what) {
  return fail(MPS_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

// The per-device word the single-tensor decode kernels OR their MPS_STATUS_*
// flags into: a module global (nothing is allocated), per device, not per stream.
int status_word(int device, uint32_t **out);

// Read a device status word and clear it, after `stream`'s work (synchronous).
int read_and_clear(int device, uint32_t *word, void *stream, const char *what, uint32_t *status_out);

}  // namespace mps

#define MPS_HIP_CHECK(expr)                                        \
  do {                                                             \
    hipError_t mps_e_ = (expr);                                    \
    if (mps_e_ != hipSuccess) return ::mps::hip_fail(mps_e_, #expr); \
  } while (0)
