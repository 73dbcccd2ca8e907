// Direct-to-LDS loads, range-checked buffer accesses and LDS reads for the
// LDS-pipelined kernels.
#pragma once

#include "common.hpp"

namespace mhc {

// ---- direct-to-LDS loads and range-checked buffer accesses -----------------
// buffer_load ... lds / global_load_lds move 16 bytes per lane to
// LDS[base + 16*lane] and count in vmcnt like any vector memory operation
// (which complete in issue order); a raw buffer access whose offset is
// beyond the resource's byte range loads zero / stores nothing.
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void glb_void_t;

constexpr uint32_t kBufferOob = 0x80000000u;  // buffer offset beyond every range

// Resource covering `bytes` bytes from `base` (raw buffer: stride 0).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rows_rsrc(const void* base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}

// s_waitcnt vmcnt(V) with the other counters left free (gfx9 encoding).
template <int V>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(V >= 0 && V < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((V & 15) | (7 << 4) | (15 << 8) | ((V >> 4) << 14));
}

// LDS byte address of a __shared__ object.
template <typename T>
__device__ __forceinline__ uint32_t lds_addr(T* p) {
  return (uint32_t)(uintptr_t)(__attribute__((address_space(3))) T*)p;
}

// LDS reads of a ring slot are inline asm the compiler does not see as LDS
// accesses (it would otherwise wait for every outstanding direct-to-LDS load,
// vmcnt(0), before each of them).  The caller orders them after the loads
// they need (wait_vmcnt + barrier).  Each asm statement issues its reads AND
// waits for them (s_waitcnt lgkmcnt(0)) before it ends: an asm output that
// the hardware writes after the statement could otherwise be copied, or its
// register reused, before the data has landed.
//   lds_read4(v, a, OFF): v[i] = 16 bytes at a + i * OFF, i = 0..3
template <int OFF>
__device__ __forceinline__ void lds_read4(u32x4 (&v)[4], uint32_t a) {
  static_assert(3 * OFF < 65536, "ds_read offset field");
  asm volatile(
      "ds_read_b128 %0, %4\n\t"
      "ds_read_b128 %1, %4 offset:%5\n\t"
      "ds_read_b128 %2, %4 offset:%6\n\t"
      "ds_read_b128 %3, %4 offset:%7\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3])
      : "v"(a), "i"(OFF), "i"(2 * OFF), "i"(3 * OFF)
      : "memory");
}

// Reads the R 1 KB units of a slot (lane's 16 bytes each), complete on return.
template <int R>
__device__ __forceinline__ void read_slot(u32x4 (&v)[R], uint32_t base) {
  static_assert(R % 4 == 1, "R = 4k + 1 rows");
#pragma unroll
  for (int i = 0; i + 4 <= R; i += 4) lds_read4<1024>(*reinterpret_cast<u32x4(*)[4]>(&v[i]), base + i * 1024);
  asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v[R - 1]) : "v"(base + (R - 1) * 1024) : "memory");
}

}  // namespace mhc
