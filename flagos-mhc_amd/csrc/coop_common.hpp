// Shared machinery of the single-pass pre kernels (pre_fwd_coop.hpp,
// pre_bwd_coop.hpp): groups of CUs on one XCC that split every 16-token tile
// by columns and exchange per-token partial sums through the XCC's L2.
//
// Group formation.  Every block (one per CU, a grid of one block per CU)
// reads its XCC from the XCC_ID hardware register and registers with a
// per-XCC counter in the control words; once all blocks have registered, an
// XCC with c blocks forms c / G groups (at most `maxg` in all) and its block
// of rank r becomes member r % G of group r / G.  Membership therefore holds
// whichever CU the dispatcher chose for a block.  Registration needs every
// block resident: a block's LDS leaves no room for a second on its CU, so on
// an otherwise idle device the whole grid is resident at once; a block that
// starts late only delays the others, and their bounded waits turn a long
// delay into a reported failure.
//
// Bounded waits.  Every wait gives up after `timeout` ticks of s_memrealtime
// (100 MHz) without progress: it raises the block's abort flag (an LDS
// counter every wait also watches) and writes its code to the status word
// (first failure wins), and every wave leaves.  The host side turns a
// nonzero status into NaN outputs and a reported error.
#pragma once

#include <atomic>

#include "lds_dma.hpp"
#include "mhc_launch.hpp"

namespace mhc {

constexpr int kCoMaxGroups = 16;
constexpr int kCoMinG = 16;  // fewest members per group
constexpr int kCoMaxG = 32;  // most members per group (CUs of an XCC)
constexpr int kCoCtlWords = 64;
constexpr uint64_t kCoTimeout = 25000000ull;  // 0.25 s of s_memrealtime (100 MHz)
// control words: [0..15] blocks registered per XCC, then the blocks that
// registered, the status word and the number of groups formed
constexpr int kCtlArrived = 16, kCtlStatus = 17, kCtlGroups = 18;
// status codes (first failure wins): 1 registration, 2 no group formed;
// each kernel numbers its own waits from 3
constexpr uint32_t kStReg = 1, kStNoGroup = 2;
// device-scope (sc1) loads: they skip this CU's L1, which may hold stale
// copies of the exchange ring, and read the XCC's L2, where the writers'
// stores land
constexpr int kCoPolicySc1 = 16;

// ---- LDS accesses (inline asm: the compiler does not see them as LDS
// operations that wait for direct-to-LDS loads, see lds_dma.hpp) and LDS
// counters ------------------------------------------------------------------
__device__ __forceinline__ uint32_t co_lds_ld(uint32_t a) {
  uint32_t v;
  asm volatile("ds_read_b32 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(a) : "memory");
  return v;
}
// No wait: a wave's LDS operations are performed in issue order, so a count
// raised after LDS writes is seen only after them, and nothing this wave
// does next depends on the add having landed.
__device__ __forceinline__ void co_lds_add(uint32_t a, uint32_t v) {
  asm volatile("ds_add_u32 %0, %1" ::"v"(a), "v"(v) : "memory");
}
__device__ __forceinline__ uint32_t co_lds_add_rtn(uint32_t a, uint32_t v) {
  uint32_t old;
  asm volatile("ds_add_rtn_u32 %0, %1, %2\n\ts_waitcnt lgkmcnt(0)" : "=v"(old) : "v"(a), "v"(v) : "memory");
  return old;
}
// Counter updates from lane 0 only: a ds_add issued by the whole wave would
// add once per active lane.  The returned old value is broadcast.
__device__ __forceinline__ void co_lds_inc(uint32_t a) {
  if (__lane_id() == 0) co_lds_add(a, 1u);
}
__device__ __forceinline__ uint32_t co_lds_inc_rtn(uint32_t a) {
  uint32_t old = 0u;
  if (__lane_id() == 0) old = co_lds_add_rtn(a, 1u);
  return __builtin_amdgcn_readfirstlane(old);
}
__device__ __forceinline__ void co_lds_st(uint32_t a, float v) {
  asm volatile("ds_write_b32 %0, %1" ::"v"(a), "v"(v) : "memory");
}
__device__ __forceinline__ void co_lds_st4(uint32_t a, floatx4 v) {  // a 16-byte aligned
  asm volatile("ds_write_b128 %0, %1" ::"v"(a), "v"(v) : "memory");
}

// A wave-uniform LDS word (a counter or flag) read into a scalar register, so
// that comparisons and loops on it are scalar branches rather than exec-mask
// manipulation.
__device__ __forceinline__ uint32_t co_lds_ld_u(uint32_t a) { return __builtin_amdgcn_readfirstlane(co_lds_ld(a)); }

__device__ __forceinline__ uint64_t co_now() { return __builtin_amdgcn_s_memrealtime(); }

__device__ __forceinline__ void co_fail(uint32_t* status, uint32_t code) {
  uint32_t expected = 0u;
  __hip_atomic_compare_exchange_strong(status, &expected, code, __ATOMIC_RELAXED, __ATOMIC_RELAXED,
                                       __HIP_MEMORY_SCOPE_AGENT);
}
// Wait until the LDS counter at `a` reaches `target` (or the block aborts /
// `timeout` ticks pass without it: then false, with the abort flag and
// status set).  A waiting wave shares its SIMD's issue slots with the waves
// doing the work, so the loop is short: it sleeps SLEEP x 64 clocks between
// reads of the counter and looks at the abort flag and the clock every
// eighth read only.
template <int SLEEP = 1>
__device__ __forceinline__ bool co_wait_ge(uint32_t a, uint32_t target, uint32_t abort_a, uint32_t* status,
                                           uint32_t code, uint64_t timeout) {
  if (co_lds_ld_u(a) >= target) return true;
  const uint64_t deadline = co_now() + timeout;
  for (uint32_t i = 1;; ++i) {
    __builtin_amdgcn_s_sleep(SLEEP);
    if (co_lds_ld_u(a) >= target) return true;
    if ((i & 7u) == 0u) {
      if (co_lds_ld_u(abort_a)) return false;
      if (co_now() > deadline) {
        co_lds_inc(abort_a);
        co_fail(status, code);
        return false;
      }
    }
  }
}

// vmcnt(n * PER) for a run-time n in [0, MAXN]
template <int PER, int MAXN>
__device__ __forceinline__ void co_wait_tiles(int n) {
  if constexpr (MAXN >= 0) {
    if (n >= MAXN) {
      wait_vmcnt<PER * MAXN>();
      return;
    }
    co_wait_tiles<PER, MAXN - 1>(n);
  }
}

// Group formation (thread 0 of a block; the caller then synchronises the
// block): info[0] = group (-1: no group), info[1] = groups formed, info[2] =
// member.  ctl: kCoCtlWords zeroed control words.
__device__ __forceinline__ void co_register(uint32_t* ctl, int G, int maxg, uint64_t timeout, int* info) {
  const uint64_t deadline0 = co_now();
  uint32_t* status = ctl + kCtlStatus;
  uint32_t xcc;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
  xcc &= 15u;
  const uint32_t rank = __hip_atomic_fetch_add(ctl + xcc, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  __hip_atomic_fetch_add(ctl + kCtlArrived, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  bool ok = true;
  while (__hip_atomic_load(ctl + kCtlArrived, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) < gridDim.x) {
    if (co_now() > deadline0 + timeout) {
      ok = false;
      break;
    }
    __builtin_amdgcn_s_sleep(2);
  }
  // an XCC with c registered blocks forms c / G groups: its block of rank r
  // is member r % G of its group r / G (if r / G < c / G)
  int group = -1, ngroups = 0;
  if (ok) {
    for (uint32_t x = 0; x < 16; ++x) {
      const uint32_t c = __hip_atomic_load(ctl + x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      const int ng = (int)(c / (uint32_t)G) < maxg - ngroups ? (int)(c / (uint32_t)G) : maxg - ngroups;
      if (x == xcc && (int)(rank / (uint32_t)G) < ng) group = ngroups + (int)(rank / (uint32_t)G);
      ngroups += ng;
    }
    if (ngroups == 0) co_fail(status, kStNoGroup);
  } else {
    co_fail(status, kStReg);
  }
  info[0] = group;
  info[1] = ngroups;
  info[2] = (int)(rank % (uint32_t)G);
}

// zero `n` 16-byte words (the control words and the exchange ring before a
// launch) with streaming stores
namespace {
__global__ __launch_bounds__(256) void co_zero_kernel(u32x4* p, int64_t n) {
  u32x4 z;
  z[0] = z[1] = z[2] = z[3] = 0u;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
    __builtin_nontemporal_store(z, p + i);
}
}  // namespace

// ---- host side --------------------------------------------------------------

// Slice geometry for D: 256-column slices, G = D / 256 members per group.
// Used where it measured faster than the two-pass forms on MI355X (32-CU
// XCCs): G = 16 (two groups per XCC, D = 4096) and 28 <= G <= 32 (one group
// per XCC, D = 7168 .. 8192).  With G = 12, 14, 20 or 24 too many CUs idle
// or the slices are too short, and the two-pass forms win; 0 selects them.
inline int coop_nch(int D, int* G) {
  if (D % 256) return 0;
  const int g = D / 256;
  if (g == 16 || (g >= 28 && g <= kCoMaxG)) {
    *G = g;
    return 32;
  }
  return 0;
}

// Groups the exchange ring is sized for: one per G CUs, at most kCoMaxGroups.
inline int coop_max_groups(int G) {
  const int g = (int)(device_cu_count() / G);
  return g < kCoMaxGroups ? g : kCoMaxGroups;
}

// Per device and kernel kind (`kind` < 4): does one block of the kernel fit a
// CU (so a grid of one block per CU is resident at once on an otherwise idle
// device), and does the kernel use no scratch memory?
inline bool coop_fits(const void* kernel, int threads, int kind) {
  static std::atomic<int> cache[64][4];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64 || kind < 0 || kind >= 4) return false;
  std::atomic<int>& slot = cache[dev][kind];
  int v = slot.load(std::memory_order_relaxed);
  if (v) return v > 0;
  int nb = 0;
  // the single-pass kernels wait on their loads with exact memory-counter
  // counts, which scratch (register spill) loads and stores issued by the
  // compiler would upset: a build with private memory does not run them
  hipFuncAttributes fa{};
  const bool ok = hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, kernel, threads, 0) == hipSuccess && nb >= 1 &&
                  hipFuncGetAttributes(&fa, kernel) == hipSuccess && fa.localSizeBytes == 0;
  (void)hipGetLastError();
  slot.store(ok ? 1 : -1, std::memory_order_relaxed);
  return ok;
}

// Limit of every bounded wait, in s_memrealtime ticks (100 MHz): kCoTimeout
// unless mhc_debug_set_wait_limit set another (a test hook that forces the
// failure path; it is never read from the environment).  One value for the
// whole process (an inline function's static).
inline std::atomic<int64_t>& coop_wait_limit_slot() {
  static std::atomic<int64_t> v{-1};
  return v;
}
inline uint64_t coop_wait_limit() {
  const int64_t v = coop_wait_limit_slot().load(std::memory_order_relaxed);
  return v < 0 ? kCoTimeout : (uint64_t)v;
}

// A stream under capture: the single-pass forms are not used there.
inline bool stream_capturing(hipStream_t st) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(st, &cs) != hipSuccess) {
    (void)hipGetLastError();
    return true;
  }
  return cs != hipStreamCaptureStatusNone;
}

}  // namespace mhc
