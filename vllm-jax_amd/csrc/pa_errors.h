// Host-side error reporting shared by the C-ABI entry points.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>

#include "../../include/paged_attention.h"

namespace pa {

// Records a formatted message for pa_last_error() and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

inline int launch_status(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(PA_ERR_LAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return PA_OK;
}

}  // namespace pa
