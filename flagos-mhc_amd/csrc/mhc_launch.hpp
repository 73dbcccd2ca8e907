// Host-side helpers shared by the C-ABI entry points: error codes, the
// thread-local error string, launch checks and alignment tests.
#pragma once

#include <hip/hip_runtime.h>
#include <stdarg.h>

#include <atomic>
#include <stdint.h>
#include <stdio.h>

#include "../../include/mhc_amd.h"

namespace mhc {

int set_error(int code, const char* fmt, ...);
void clear_error();

inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Compute units of the current device, queried once per device (safe to call
// from several host threads; a failed query reads as 256, the MI355X count).
inline int device_cu_count() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  int cus = cache[dev].load(std::memory_order_relaxed);
  if (cus > 0) return cus;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    cus = 256;
  cache[dev].store(cus, std::memory_order_relaxed);
  return cus;
}

// Dynamic LDS bytes that keep a kernel at one block per CU: just over half
// of a CU's LDS (a kernel that uses no LDS of its own then never shares its
// CU with a second block).  The streaming kernels that read a token's rows
// as contiguous runs are faster with fewer tokens in flight per CU.  Queried
// once per device; 0 if the device does not report its LDS sizes.
inline size_t one_block_per_cu_lds() {
  static std::atomic<long long> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  long long v = cache[dev].load(std::memory_order_relaxed);
  if (v > 0) return (size_t)(v - 1);
  int per_cu = 0, per_block = 0;
  size_t pad = 0;
  if (hipDeviceGetAttribute(&per_cu, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev) == hipSuccess &&
      hipDeviceGetAttribute(&per_block, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) == hipSuccess &&
      per_cu > 0 && per_block > per_cu / 2)
    pad = (size_t)(per_cu / 2 + 1024);
  if (pad > (size_t)per_block) pad = 0;
  cache[dev].store((long long)pad + 1, std::memory_order_relaxed);
  return pad;
}

// Token counts above this are refused: several grids put one block (or one
// per 16 tokens) in a 32-bit grid dimension, which must not wrap.
constexpr int64_t kMaxTokens = 2147483647;

// A dispatch packet holds the grid size in work-items as 32-bit numbers, so a
// grid of one block per token of B threads fits up to (2^32 - 1) / B tokens
// (4.2 M with 1024-thread blocks).  Launches of that form check it first and
// refuse larger calls instead of relying on the runtime.
inline int check_grid(const dim3& g, const dim3& b, const char* what) {
  const uint64_t lim = 0xffffffffull;
  if ((uint64_t)g.x * b.x > lim || (uint64_t)g.y * b.y > lim || (uint64_t)g.z * b.z > lim)
    return set_error(MHC_ERR_UNSUPPORTED, "%s: %u x %u x %u blocks of %u x %u x %u threads exceed the 2^32 work-items of a dispatch",
                     what, g.x, g.y, g.z, b.x, b.y, b.z);
  return MHC_OK;
}

inline int check_tokens(int64_t T, const char* who) {
  if (T > kMaxTokens)
    return set_error(MHC_ERR_UNSUPPORTED, "%s: T=%lld above the supported %lld tokens", who, (long long)T,
                     (long long)kMaxTokens);
  return MHC_OK;
}

// Reports a failed launch (bad configuration, missing code object, ...).
inline int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess)
    return set_error(MHC_ERR_HIP, "%s: kernel launch failed: %s", what, hipGetErrorString(e));
  return MHC_OK;
}

}  // namespace mhc
