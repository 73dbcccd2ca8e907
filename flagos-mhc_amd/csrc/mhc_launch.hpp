// Host-side helpers shared by the C-ABI entry points: error codes, the
// thread-local error string, launch checks and alignment tests.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/mhc_amd.h"

namespace mhc {

int set_error(int code, const char* fmt, ...);
void clear_error();

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Reports a failed launch (bad configuration, missing code object, ...).
inline int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(MHC_ERR_HIP, "%s: kernel launch failed: %s", what, hipGetErrorString(e));
  return MHC_OK;
}

}  // namespace mhc
