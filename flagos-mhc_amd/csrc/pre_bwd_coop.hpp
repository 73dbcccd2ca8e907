// mhc_pre_clamp_sinkhorn backward in one HBM pass over x and grad_y: N = 4,
// bf16 x, grad_y and phi, D = 256 G with the forward's slice geometry
// (coop_nch: G = 16 or 28 <= G <= 32).  Included by pre_bwd.hip.
//
// Semantics: torch autograd of mhc_pre_clamp_sinkhorn_ref, as the
// reference's mhc_pre_clamp_sinkhorn_backward_ref
// (src/mhc_pre_clamp_sinkhorn_backward.py:1397-1453).  The passes it replaces
// are the reference's grad_pre pass (_y_bwd_kernel_hc4, :68-155) and its
// rms-backward / combine pass (_fused_ybwd_rmsbwd_kernel, :217-341, with the
// two torch.mm of :1372-1373), which read x and grad_y twice.
//
// Only the pre head's part of grad_mixes needs grad_pre[t, n] = <grad_y[t],
// x[t, n]>, a reduction over the whole N*D row of a token:
//   grad_mixes[t, n] = grad_pre[t, n] * alpha[0] * sp (1 - sp)  (n < 4)
// the other 20 entries, the Sinkhorn / softmax / clamp and post-head VJPs,
// come from kernel A (pre_bwd_small_kernel, SP form) before this kernel,
// with the per-token record coefX (pre, sp (1 - sp), mixes[0..3], inv_rms,
// the scale without the pre head).  Then
//   grad_x[t, n, d] = grad_y[t, d] pre[t, n] + inv[t] gs[t, n, d] + scale[t] x[t, n, d]
//   gs = grad_mixes @ phi,  scale = -inv^2 <grad_mixes, mixes> / (N D)
//   grad_phi += (grad_mixes inv)^T @ x
// all need that row reduction finished before a column of the row can be
// written.  So, as in the single-pass forward, G CUs of one XCC form a group
// that shares every 16-token tile: member c owns columns [256 c, 256 c + 256)
// of the four streams (32 KB of x and 8 KB of grad_y per tile) and keeps them
// on chip from their one HBM read until grad_x of those columns is written.
//
// A block (one per CU) has four waves, wave n owning stream n's 256 columns
// of the slice; lane (r, q) holds tokens 4 q .. 4 q + 3 and columns 8 r ..
// 8 r + 7 of each 128-column half (the lane layout of the two-pass kernel B,
// pre_bwd_dma_kernel).  Per iteration j (tile j landing, tile u = j - 2 in
// phase 2):
//   * direct-to-LDS loads of tile j + 2: x into 3 slots of 32 KB, grad_y,
//     kernel A's grad_mixes rows and records into 4 slots of 10.5 KB;
//   * phase 1 of tile j: copy its x into a ring of two tiles of registers
//     (freeing the slot) and sum grad_y . x per token over the wave's
//     columns (v_dot2_f32_bf16), then over the 16 lanes of a row (DPP); the
//     member's record of the tile (16 tokens x 4 streams as 4 chunks of 8
//     16-byte words, word w of a chunk (value w, value w + 8, tag, tag))
//     goes to the group's ring, each wave storing the 8 words that hold its
//     stream's sums;
//   * exchange of tile u: wave w polls chunk w of every member's record (4
//     direct-to-LDS loads, lane = (member, word)), adds over members in a
//     fixed order, forms its four tokens' grad_mixes[0..3] and scale, and
//     writes its share of the tile's phase-2 operands that all four waves
//     use (g = grad_mixes inv in both bf16 planes as MFMA A operands, the
//     diagonal words of pre and scale) to LDS, once for the block;
//   * phase 2 of tile u: grad_phi partial += g^T @ x and grad_x = diag(pre)
//     grad_y + diag(scale) x + (grad_mixes inv) @ phi on the matrix cores
//     (16x16x32 MFMAs, both bf16 planes of each fp32 factor), grad_x stored
//     once.
// The records are the only data that cross CUs (512 bytes per member and
// tile), and they stay in the XCC's L2: the tag (tile sequence + 1) in every
// 16-byte word tells a reader that the word has arrived; a word is written
// by one store and read by one load, so it never tears.  Each group writes
// its own grad_phi partial [group][M][K]; the member that owns a tile (tile
// sequence % G) adds the tile's grad_alpha[0] / grad_base[0..3] terms to its
// row of contributions.  Both are summed in fixed order afterwards
// (deterministic; no atomics on data).
//
// Memory-counter accounting.  Vector memory operations complete in issue
// order; each wave waits for a tile's loads and for its poll with s_waitcnt
// vmcnt(n), n the exact number of operations it issued after them in the
// steady state (vmcnt(0) near the ends of the loop).  That needs a build
// without scratch memory (no spill loads or stores among them): the host
// side runs the kernel only when its private segment is empty.
#pragma once

#include "coop_common.hpp"

namespace mhc {

constexpr int kBcTT = 16;                 // tokens per tile
constexpr int kBcWaves = 4;               // one per stream
constexpr int kBcLag = 2;                 // phase 2 of tile j - 2 while tile j lands
constexpr int kBcSx = 3;                  // x slots of 32 KB
constexpr int kBcSg = 4;                  // grad_y / per-token slots of 10.5 KB
constexpr int kBcGSlot = 10752;           // grad_y (8 KB) + coefX (1 KB) + grad_mixes rows (1.5 KB)
constexpr int kBcCoef = 8 * 1024;         // offset of coefX in a grad_y slot
constexpr int kBcGm = 9 * 1024;           // offset of the grad_mixes rows [16][24] fp32
// The shared phase-2 operands of a tile (opw, bytes): the A operands of the
// grad_mixes @ phi product (hi / lo planes, lane (r, q): token r, m = 8 q ..
// 8 q + 7), of the grad_phi products (rows m = 16 mt + r, lane (r, q): tokens
// 4 q .. 4 q + 3, both planes), and the diagonal words (hi | lo << 16) of
// pre[16][4] and scale[16]; entries no wave writes (m >= 24) stay zero.
constexpr int kBcOpA0 = 0, kBcOpA1 = 1024, kBcOpT0 = 2048, kBcOpT1 = 3072, kBcOpPre = 4096, kBcOpSc = 4352;
constexpr int kBcOpBytes = 4416;
constexpr int kBcR = 16;                  // exchange ring: tiles per group
constexpr int kBcChunkWords = 8;          // a record chunk: 16 sums (4 tokens x 4 streams), word w = (v_w, v_{w+8}, tag, tag)
constexpr int kBcRecWords = 4 * kBcChunkWords;  // a member's record of a tile: 4 chunks
constexpr int kBcPollKB = kCoMaxG * kBcChunkWords / 64;  // a wave's poll buffer, 1 KB units (4): 8 members each
constexpr int kBcMaxGroups = kCoMaxGroups;
constexpr int kBcThreads = kBcWaves * kWave;
// status codes: the wait that timed out
constexpr uint32_t kBcStPoll = 7;
static_assert(kBcR >= 2 * kBcLag + 4, "exchange ring shorter than the skew it must cover");
static_assert((kBcR & (kBcR - 1)) == 0 && (kBcSg & (kBcSg - 1)) == 0, "slot indices are masks");

struct BwdCoopArgs {
  const bf16_t* x;       // (T, 4, D)
  const bf16_t* gy;      // (T, D)
  bf16_t* gx;            // (T, 4, D)
  const uint16_t* phiT;  // [K][32] bf16, m padded to 32 with zeros
  const float* gm;       // (T, 24) grad_mixes without the pre head (kernel A, SP form)
  const float* coefX;    // (T, 16) per-token records of kernel A
  const float* alpha;
  float* part;           // [maxg][24][K] grad_phi partial of each group
  float* contrib;        // [maxg * G][27] grad_alpha / grad_base terms of each member (zeroed before the launch)
  uint32_t* ctl;         // kCoCtlWords control words, zeroed before the launch
  u32x4* rec;            // [maxg][kBcR][4 chunks][G][kBcChunkWords], zeroed before the launch
  int64_t T;
  int D;
  int G;
  int maxg;
  uint64_t timeout;
};

// s_waitcnt vmcnt(BASE + kg) for wave-uniform kg in {2, 3}: the
// steady-state counts of the main loop's two waits
template <int BASE>
__device__ __forceinline__ void bc_wait_steady(int kg) {
  static_assert(BASE + 3 < 64, "vmcnt range");
  if (kg == 3)
    wait_vmcnt<BASE + 3>();
  else
    wait_vmcnt<BASE + 2>();
}

// An opaque copy of a wave-uniform value: what derives from it (LDS slot and
// counter addresses) is recomputed where it is used, a scalar add, instead of
// every derived value being kept live across the main loop, where the
// scalar registers run out and the values go to VGPR lanes.
__device__ __forceinline__ uint32_t bc_opq(uint32_t v) {
  asm volatile("" : "+s"(v));
  return v;
}

// Block barrier after this wave's LDS operations have completed; memory
// loads in flight (the direct-to-LDS ring) are left running.
__device__ __forceinline__ void bc_sync() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// c + a.lo b.lo + a.hi b.hi for two bf16 pairs (v_dot2c_f32_bf16: the bf16
// products are exact in fp32)
__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a), __builtin_bit_cast(bf16x2_t, b), c, false);
}

// Phase 1: the lane's x of both halves (8 units from xa, 1 KB apart) and
// grad_y of both halves (4 units from g0 and 4 from g0 + 4 KB), one wait.
__device__ __forceinline__ void bc_rd_phase1(u32x4 (&x)[2][4], u32x4 (&g)[2][4], uint32_t xa, uint32_t ga) {
  asm volatile(
      "ds_read_b128 %0, %16\n\t"
      "ds_read_b128 %1, %16 offset:1024\n\t"
      "ds_read_b128 %2, %16 offset:2048\n\t"
      "ds_read_b128 %3, %16 offset:3072\n\t"
      "ds_read_b128 %4, %16 offset:4096\n\t"
      "ds_read_b128 %5, %16 offset:5120\n\t"
      "ds_read_b128 %6, %16 offset:6144\n\t"
      "ds_read_b128 %7, %16 offset:7168\n\t"
      "ds_read_b128 %8, %17\n\t"
      "ds_read_b128 %9, %17 offset:1024\n\t"
      "ds_read_b128 %10, %17 offset:2048\n\t"
      "ds_read_b128 %11, %17 offset:3072\n\t"
      "ds_read_b128 %12, %17 offset:4096\n\t"
      "ds_read_b128 %13, %17 offset:5120\n\t"
      "ds_read_b128 %14, %17 offset:6144\n\t"
      "ds_read_b128 %15, %17 offset:7168\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(x[0][0]), "=&v"(x[0][1]), "=&v"(x[0][2]), "=&v"(x[0][3]), "=&v"(x[1][0]), "=&v"(x[1][1]),
        "=&v"(x[1][2]), "=&v"(x[1][3]), "=&v"(g[0][0]), "=&v"(g[0][1]), "=&v"(g[0][2]), "=&v"(g[0][3]),
        "=&v"(g[1][0]), "=&v"(g[1][1]), "=&v"(g[1][2]), "=&v"(g[1][3])
      : "v"(xa), "v"(ga)
      : "memory");
}

// Phase 2's operands in one batch of reads: the shared A operands at oa
// (kBcOpA0 / A1 / T0 / T1 from the tile's opw), the diagonal words of pre[r][n]
// and scale[r] (pa, sa), and the lane's grad_y units of both halves (g1:
// half 1, g0: half 0, 1 KB apart); one wait.
__device__ __forceinline__ void bc_rd_ops(u32x4& a0, u32x4& a1, u32x4& t0, u32x4& t1, uint32_t& pw, uint32_t& sw,
                                          u32x4 (&g1)[4], u32x4 (&g0)[4], uint32_t oa, uint32_t pa, uint32_t sa,
                                          uint32_t ga1, uint32_t ga0) {
  static_assert(kBcOpA0 == 0 && kBcOpA1 == 1024 && kBcOpT0 == 2048 && kBcOpT1 == 3072, "offsets below");
  asm volatile(
      "ds_read_b128 %0, %14\n\t"
      "ds_read_b128 %1, %14 offset:1024\n\t"
      "ds_read_b128 %2, %14 offset:2048\n\t"
      "ds_read_b128 %3, %14 offset:3072\n\t"
      "ds_read_b32 %4, %15\n\t"
      "ds_read_b32 %5, %16\n\t"
      "ds_read_b128 %6, %17\n\t"
      "ds_read_b128 %7, %17 offset:1024\n\t"
      "ds_read_b128 %8, %17 offset:2048\n\t"
      "ds_read_b128 %9, %17 offset:3072\n\t"
      "ds_read_b128 %10, %18\n\t"
      "ds_read_b128 %11, %18 offset:1024\n\t"
      "ds_read_b128 %12, %18 offset:2048\n\t"
      "ds_read_b128 %13, %18 offset:3072\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(a0), "=&v"(a1), "=&v"(t0), "=&v"(t1), "=&v"(pw), "=&v"(sw), "=&v"(g1[0]), "=&v"(g1[1]), "=&v"(g1[2]),
        "=&v"(g1[3]), "=&v"(g0[0]), "=&v"(g0[1]), "=&v"(g0[2]), "=&v"(g0[3])
      : "v"(oa), "v"(pa), "v"(sa), "v"(ga1), "v"(ga0)
      : "memory");
}

// The A operand of a 16x16x32 MFMA holding diag(v) over a tile's 16 tokens in
// both bf16 planes (k = 8 q + 2 e + p: token 4 q + e, plane p; paired with a
// bc_col2 B operand) from v's word w = hi | lo << 16: lane (r, q) holds row r,
// so only the lane with q == r / 4 has a nonzero dword, e = r % 4.
__device__ __forceinline__ u32x4 bc_diagw(uint32_t w, int r, int q) {
  const uint32_t d = q == (r >> 2) ? w : 0u;
  const int e = r & 3;
  return u32x4{e == 0 ? d : 0u, e == 1 ? d : 0u, e == 2 ? d : 0u, e == 3 ? d : 0u};
}

// v's two bf16 planes as one word, hi | lo << 16 (the dword of a diagonal or
// grad_phi A operand)
__device__ __forceinline__ uint32_t bc_word2(float v) {
  uint32_t hi, lo;
  split2_bf16(v, hi, lo);
  return hi | (lo << 16);
}

// Column c of a lane's 4-token x 8-column block of bf16 (m[e][c / 2] holds
// columns 2 (c / 2), + 1 of token e) as the B operand of a 16x16x32 MFMA
// whose k = 2 e + p runs over the lane's tokens e and two planes p of the A
// operand: dword e = the token's value twice.
__device__ __forceinline__ u32x4 bc_col2(const u32x4 (&m)[4], int C) {
  const uint32_t sel = (C & 1) ? 0x03020302u : 0x01000100u;
  const int w = C >> 1;
  return u32x4{__builtin_amdgcn_perm(m[0][w], m[0][w], sel), __builtin_amdgcn_perm(m[1][w], m[1][w], sel),
               __builtin_amdgcn_perm(m[2][w], m[2][w], sel), __builtin_amdgcn_perm(m[3][w], m[3][w], sel)};
}

// The poll buffer's four 1 KB units (the lane's 16 bytes of each, at pa)
// and five 4-byte reads (pre, cz, mix, inv, scale without the pre head), one
// wait
__device__ __forceinline__ void bc_rd_poll(u32x4 (&p)[4], float& pre, float& cz, float& mix, float& inv, float& sk,
                                           uint32_t pa, uint32_t ca, uint32_t cb) {
  uint32_t v[5];
  asm volatile(
      "ds_read_b128 %0, %9\n\t"
      "ds_read_b128 %1, %9 offset:1024\n\t"
      "ds_read_b128 %2, %9 offset:2048\n\t"
      "ds_read_b128 %3, %9 offset:3072\n\t"
      "ds_read_b32 %4, %10\n\t"
      "ds_read_b32 %5, %10 offset:16\n\t"
      "ds_read_b32 %6, %10 offset:32\n\t"
      "ds_read_b32 %7, %11 offset:48\n\t"
      "ds_read_b32 %8, %11 offset:52\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(p[0]), "=&v"(p[1]), "=&v"(p[2]), "=&v"(p[3]), "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]),
        "=&v"(v[4])
      : "v"(pa), "v"(ca), "v"(cb)
      : "memory");
  pre = __uint_as_float(v[0]);
  cz = __uint_as_float(v[1]);
  mix = __uint_as_float(v[2]);
  inv = __uint_as_float(v[3]);
  sk = __uint_as_float(v[4]);
}

// One 8-byte read (the grad_mixes rows' pair at a, 8-byte aligned) and one
// 4-byte read (the word at b), one wait
__device__ __forceinline__ void bc_rd_pair(float& x0, float& x1, float& y, uint32_t a, uint32_t b) {
  u32x2 v;
  uint32_t w;
  asm volatile(
      "ds_read_b64 %0, %2\n\t"
      "ds_read_b32 %1, %3\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(v), "=&v"(w)
      : "v"(a), "v"(b)
      : "memory");
  x0 = __uint_as_float(v[0]);
  x1 = __uint_as_float(v[1]);
  y = __uint_as_float(w);
}

__global__ __launch_bounds__(kBcThreads) void pre_bwd_coop_kernel(BwdCoopArgs a) {
  constexpr int M = 24, C = 3 + M;
  __shared__ __align__(1024) u32x4 xs[kBcSx * 32 * kWave];           // 96 KB: [slot][stream][h][e] 1 KB units
  __shared__ __align__(1024) u32x4 gsl[kBcSg * kBcGSlot / 16];       // 42 KB
  __shared__ __align__(1024) u32x4 pbuf[kBcWaves * kBcPollKB * kWave];  // 16 KB: each wave's poll
  __shared__ __align__(16) uint32_t opw[kBcOpBytes / 4];             // the shared phase-2 operands
  __shared__ __align__(16) float red[kBcWaves][8];                   // end: the waves' contributions
  // counters: abort at 22
  __shared__ uint32_t cnt[32];
  __shared__ int info[4];

  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // = stream n
  const int n = wave;
  const int r = lane & 15, q = lane >> 4;
  const int64_t T = a.T;
  const int D = a.D, G = a.G;
  const int64_t K = 4 * (int64_t)D;
  const uint64_t to = a.timeout;
  uint32_t* status = a.ctl + kCtlStatus;

  if (tid < 32) cnt[tid] = 0u;
  // the operand entries of m >= 24 are never written: zero for every tile
  for (int i = tid; i < kBcOpBytes / 4; i += kBcThreads) opw[i] = 0u;
  if (tid == 0) co_register(a.ctl, G, a.maxg, to, info);
  __syncthreads();
  const int group = info[0], ngroups = info[1], member = info[2];
  if (group < 0) return;  // uniform over the block: not a member of a group
  if (tid == 0) __hip_atomic_store(a.ctl + kCtlGroups, (uint32_t)ngroups, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // tile and loop indices fit 32 bits (the host bounds T)
  const int ntiles = (int)((T + kBcTT - 1) / kBcTT);
  const int nqr = (ntiles - group + ngroups - 1) / ngroups;  // tiles of this group
  const int nq = nqr > 0 ? nqr : 0;
  const int slice0 = member * 256;
  u32x4* recw = a.rec + (size_t)group * kBcR * G * kBcRecWords;
  const auto ring = rows_rsrc(recw, (int64_t)kBcR * G * kBcRecWords * 16);
  const uint32_t xs_l = lds_addr(xs), gs_l = lds_addr(gsl), pb_l = lds_addr(pbuf) + wave * kBcPollKB * 1024;
  const uint32_t opw_l = lds_addr(opw);
  const uint32_t c_ab = lds_addr(cnt) + 88;
  const int kg = wave < 3 ? 3 : 2;  // grad_y / per-token loads this wave issues per tile
  constexpr int npoll = kBcPollKB;  // poll loads a wave issues per tile
  const float a0 = __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(a.alpha[0])));
  const float invK = 1.0f / (float)K;
  auto t0_of = [&](int qi) { return (int64_t)(group + qi * ngroups) * kBcTT; };
  auto nv_of = [&](int64_t t0) { return (int)(T - t0 < kBcTT ? T - t0 : kBcTT); };
  // ---- loads: tile qi's x units of this stream (8), its grad_y units (h, e =
  // wave) and (waves 0..2) a third of the per-token data: wave 0 grad_mixes
  // bytes [0, 1024), wave 1 [1024, 1536) (lanes past 1536 read zeros into the
  // slot's padding), wave 2 coefX
  auto issue_x = [&](int qi) {
    const int64_t t0 = t0_of(qi);
    const int nv = nv_of(t0);
    const auto rx = rows_rsrc(a.x + (t0 * 4 + n) * (int64_t)D + slice0, ((int64_t)(nv - 1) * K + 256) * 2);
    const uint32_t slot = bc_opq(xs_l) + ((uint32_t)qi % (uint32_t)kBcSx) * 32 * 1024 + (uint32_t)n * 8192;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh)
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int tok = 4 * q + e;
        const uint32_t off = tok < nv ? (uint32_t)(((int64_t)tok * K + 128 * hh + 8 * r) * 2) : kBufferOob;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_void_t*)(uintptr_t)(slot + (hh * 4 + e) * 1024), 16, off,
                                                 0, 0, 2 /* nt */);
      }
  };
  auto issue_g = [&](int qi) {
    const int64_t t0 = t0_of(qi);
    const int nv = nv_of(t0);
    const uint32_t slot = bc_opq(gs_l) + (uint32_t)(qi & (kBcSg - 1)) * kBcGSlot;
    const auto rg = rows_rsrc(a.gy + t0 * D + slice0, ((int64_t)(nv - 1) * D + 256) * 2);
    const int tok = 4 * q + wave;
#pragma unroll
    for (int hh = 0; hh < 2; ++hh) {
      const uint32_t off = tok < nv ? (uint32_t)(((int64_t)tok * D + 128 * hh + 8 * r) * 2) : kBufferOob;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rg, (lds_void_t*)(uintptr_t)(slot + (4 * hh + wave) * 1024), 16,
                                               off, 0, 0, 2 /* nt */);
    }
    if (wave < 2) {
      // wave 1: the 512 bytes past the first 1 KB, from lanes 0..31 (the
      // others are masked off and write nothing)
      const auto rm = rows_rsrc(a.gm + t0 * M, (int64_t)nv * M * 4);
      if (wave == 0 || lane < 32)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rm, (lds_void_t*)(uintptr_t)(slot + kBcGm + wave * 1024), 16,
                                                 (uint32_t)(wave * 1024 + 16 * lane), 0, 0, 0);
    } else if (wave == 2) {
      const auto rc = rows_rsrc(a.coefX + t0 * 16, (int64_t)nv * 64);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rc, (lds_void_t*)(uintptr_t)(slot + kBcCoef), 16,
                                               (uint32_t)(16 * lane), 0, 0, 0);
    }
  };
  // ---- poll: chunk `wave` of every member's record of tile u into this
  // wave's poll buffer (member i's word w at (6 i + w) * 16) ----------------
  auto issue_poll = [&](int u) {
#pragma unroll
    for (int k = 0; k < npoll; ++k) {
      // lane l: word l % 8 of member 8 k + l / 8 (members past G read zeros)
      const int f = 64 * k + lane, i = f / kBcChunkWords;
      const uint32_t off =
          i < G ? (uint32_t)((((u & (kBcR - 1)) * 4 + wave) * G * kBcChunkWords + f) * 16) : kBufferOob;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ring, (lds_void_t*)(uintptr_t)(bc_opq(pb_l) + k * 1024), 16, off, 0, 0,
                                               kCoPolicySc1);
    }
  };

  // phi^T operands of the lane's columns (B of gs: m = 8 q .. 8 q + 7) and the
  // grad_phi accumulators (rows 16 mt + 4 q + v, column c of the lane's 8 in
  // half h)
  u32x4 pb[2][8];
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    const int64_t kcol = (int64_t)n * D + slice0 + 128 * hh + 8 * r;
#pragma unroll
    for (int c = 0; c < 8; ++c) pb[hh][c] = ld16(a.phiT + (kcol + c) * 32 + 8 * q);
  }
  floatx4 ph[2][2][8];
#pragma unroll
  for (int hh = 0; hh < 2; ++hh)
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int c = 0; c < 8; ++c) ph[hh][mt][c] = floatx4{0.f, 0.f, 0.f, 0.f};
  float acc_c0 = 0.f, acc_b = 0.f;  // the owner's grad_alpha[0] / grad_base[n] terms
  wait_vmcnt<0>();  // phi operands in registers before any direct-to-LDS load is issued
  asm volatile("" ::: "memory");

  // prologue, in the order the loop would have issued them (a tile's grad_y
  // loads before its x loads)
  if (nq > 0) issue_g(0);
  if (nq > 0) issue_x(0);
  if (nq > 1) issue_g(1);
  if (nq > 1) issue_x(1);

  int own = 0;  // (tile u) % G: the member that owns tile u's grad_alpha / grad_base terms
  // Iteration j, with u = j - 2:
  //   (E) this wave's share of the exchange of tile u (chunk `wave`: tokens
  //       4 wave .. 4 wave + 3), (F) wait for all four shares, (H) phase 2
  //       of tile u from Xr with its stores, (G) this wave's poll of tile
  //       u + 1,
  //   (A) tile j landed, (B) phase 1 of tile j into Xr (the registers phase
  //       2 just released), (D) this wave's words of the record of tile j,
  //       (C) tile j + 2's grad_y loads into tile u's slot and its x loads.
  // So only two tiles of x sit in registers at a time.  The poll is issued
  // before this iteration's loads, so it completes after older work only.
  // Every index is a 32-bit scalar; every wait on a counter is a
  // scalar branch.  A wait that gives up (abort flag and status set) lets
  // the loop run to its end on whatever the buffers hold (every later wait
  // returns at once, and the loads and stores stay in range); the sum
  // kernel then replaces the outputs with NaN.  Block barriers order
  // the waves ((F): the exchange results ready; (A): tile j landed and
  // every wave done with phase 2 of tile u, which frees its grad_y slot
  // and, for tile u + 1, the operands' buffer, and with every buffer
  // iteration j - 1 read); every wave runs the same iterations, so each
  // barrier is reached by all four (the bounded waits end, failed or not).
  auto step = [&](int j, u32x4 (&Xr)[2][4]) {
    const int u = j - kBcLag;
    if (u >= 0 && u < nq) {
      const uint32_t gslot = bc_opq(gs_l) + (uint32_t)(u & (kBcSg - 1)) * kBcGSlot;
      // ---- (E) this wave's share of the exchange of tile u -------------------
      {
        // operations issued after the poll (iteration j - 1: this wave's
        // words of the record of tile j - 1 (1), grad_y loads of tile j + 1
        // (kg), x loads of tile j + 1 (8)); away from the steady state all of
        // them
        if (j >= 3 && j + 1 < nq)
          bc_wait_steady<9>(kg);
        else
          wait_vmcnt<0>();
        const uint32_t tag = (uint32_t)(u + 1);
        uint64_t deadline = 0;
        float s0, s1;
        // lane v < 16 of the chunk: token t = 4 wave + v / 4, stream v % 4
        const int t = 4 * wave + ((lane & 15) >> 2), nn = lane & 3;
        const uint32_t cf = gslot + kBcCoef + (uint32_t)(t * 64);
        float pre, cz, mix, inv, sk;
        for (;;) {
          // lane l: word w = l % 8 of members l / 8 + 8 k, k = 0..3; every
          // valid word of the G members must carry this tile's tag
          u32x4 v[4];
          bc_rd_poll(v, pre, cz, mix, inv, sk, bc_opq(pb_l) + (uint32_t)(16 * lane), cf + 4 * nn, cf);
          uint32_t cur = 0;
#pragma unroll
          for (int k = 0; k < 4; ++k) cur += (uint32_t)__popcll(__ballot(v[k][2] == tag));
          if (cur == (uint32_t)(kBcChunkWords * G)) {
            // members past G are zeros; the sum runs over k, then over the
            // lanes of the same word (l ^ 8, l ^ 16, l ^ 32): a fixed order
            s0 = (__uint_as_float(v[0][0]) + __uint_as_float(v[1][0])) + (__uint_as_float(v[2][0]) + __uint_as_float(v[3][0]));
            s1 = (__uint_as_float(v[0][1]) + __uint_as_float(v[1][1])) + (__uint_as_float(v[2][1]) + __uint_as_float(v[3][1]));
            s0 = group_sum<56>(s0);
            s1 = group_sum<56>(s1);
            break;
          }
          s0 = s1 = 0.f;
          if (deadline == 0) deadline = co_now() + to;
          if (co_lds_ld_u(bc_opq(c_ab))) break;
          if (co_now() > deadline) {
            co_lds_inc(bc_opq(c_ab));
            co_fail(status, kBcStPoll);
            break;
          }
          __builtin_amdgcn_s_sleep(1);
          issue_poll(u);
          wait_vmcnt<0>();
        }
        // lane v < 16 holds word v % 8 of the chunk, whose components are
        // values v % 8 and v % 8 + 8: value v is component v / 8
        const float gp = (lane & 8) ? s1 : s0;
        const float gz = gp * cz;
        const float gmv = gz * a0;
        const float sd = group_sum<3>(gmv * mix);
        const float sc = sk - inv * inv * sd * invK;
        // The tile's shared phase-2 operands for this wave's tokens 4 wave ..
        // 4 wave + 3 (opw held tile u - 1's: every wave finished phase 2 of
        // it before the barrier of (A) in the last iteration).  Lane l forms
        // g = grad_mixes * inv of token rt = 4 wave + l / 16 at m0 = 8 fq +
        // 2 fp and m0 + 1 (fq = l / 4 % 4, fp = l % 4; m < 4 from the
        // exchange, whose value (token rt, m) every 16 lanes hold at lane
        // 4 (l / 16) + m), and writes both planes into the A operands of the
        // grad_mixes @ phi product (lane (rt, fq)) and of the grad_phi
        // product (rows m: lane (m % 16, wave), dword l / 16)
        {
          const uint32_t ob = bc_opq(opw_l);
          const int tl = lane >> 4, fq = (lane >> 2) & 3, fp = lane & 3;
          const int m0 = 8 * fq + 2 * fp, rt = 4 * wave + tl;
          const float e0 = __int_as_float(__builtin_amdgcn_ds_bpermute(4 * (4 * tl + (m0 & 3)), __float_as_int(gmv)));
          const float e1 = __int_as_float(__builtin_amdgcn_ds_bpermute(4 * (4 * tl + (m0 & 3) + 1), __float_as_int(gmv)));
          float g0, g1, ir;
          bc_rd_pair(g0, g1, ir, gslot + kBcGm + (uint32_t)((rt * M + (m0 < M ? m0 : 0)) * 4),
                     gslot + kBcCoef + (uint32_t)(rt * 64 + 48));
          const float s0 = m0 < 4 ? e0 : g0, s1 = m0 < 4 ? e1 : g1;
          float f0 = s0 * ir, f1 = s1 * ir;
          const uint32_t h0 = f32_to_bf16_bits(f0), h1 = f32_to_bf16_bits(f1);
          if (fq < 3) {
            // lo plane of the gs operand: the residual of the exact product
            // (one fma)
            const uint32_t l0 = f32_to_bf16_bits(fmaf(s0, ir, -bf16_bits_to_f32(h0)));
            const uint32_t l1 = f32_to_bf16_bits(fmaf(s1, ir, -bf16_bits_to_f32(h1)));
            const uint32_t aa = ob + (uint32_t)(16 * (16 * fq + rt) + 4 * fp);
            co_lds_st(aa + kBcOpA0, __uint_as_float(h0 | (h1 << 16)));
            co_lds_st(aa + kBcOpA1, __uint_as_float(l0 | (l1 << 16)));
          }
          if (m0 < M) {
            // lo plane of the grad_phi operand: the residual of the rounded
            // product (kept opaque, so no fma forms)
            asm volatile("" : "+v"(f0), "+v"(f1));
            const uint32_t l0 = f32_to_bf16_bits(f0 - bf16_bits_to_f32(h0));
            const uint32_t l1 = f32_to_bf16_bits(f1 - bf16_bits_to_f32(h1));
            // m0 and m0 + 1 share a row block (m0 is even): lanes m0 % 16 and + 1
            const uint32_t ta = ob + kBcOpT0 + (uint32_t)((m0 >> 4) * 1024 + 16 * ((m0 & 15) + 16 * wave) + 4 * tl);
            co_lds_st(ta, __uint_as_float(h0 | (l0 << 16)));
            co_lds_st(ta + 16, __uint_as_float(h1 | (l1 << 16)));
          }
          if (lane < 16) {
            co_lds_st(ob + kBcOpPre + (uint32_t)(4 * (4 * t + nn)), __uint_as_float(bc_word2(pre)));
            if (nn == 0) co_lds_st(ob + kBcOpSc + (uint32_t)(4 * t), __uint_as_float(bc_word2(sc)));
          }
        }
        const bool owner = own == member;  // the tile's owner adds its grad_alpha[0] / grad_base terms
        if (owner && lane < 16) {
          acc_c0 = fmaf(gz, mix, acc_c0);
          acc_b += gz;
        }
      }
      // ---- (F) wait for the four shares -------------------------------------
      bc_sync();
    }
    if (u >= 0 && u < nq) {
      // ---- (H) phase 2 of tile u --------------------------------------------
      const uint32_t gslot = bc_opq(gs_l) + (uint32_t)(u & (kBcSg - 1)) * kBcGSlot;
      // operands: gA = grad_mixes * inv of token r, m = 8 q .. 8 q + 7 (hi /
      // lo planes); gt[mt] = g = grad_mixes * inv of row m = 16 mt + r for
      // tokens 4 q .. 4 q + 3 (dword e: token e's hi and lo planes);
      // diag(pre[., n]) and diag(scale) over the tile's tokens; grad_y of
      // both halves
      u32x4 gA0, gA1, gt[2], grh[2][4], dpre, dsc;
      {
        const uint32_t ob = bc_opq(opw_l);
        uint32_t pw, sw;
        bc_rd_ops(gA0, gA1, gt[0], gt[1], pw, sw, grh[1], grh[0], ob + (uint32_t)(16 * lane),
                  ob + kBcOpPre + (uint32_t)(4 * (4 * r + n)), ob + kBcOpSc + (uint32_t)(4 * r),
                  gslot + (uint32_t)(4096 + 16 * lane), gslot + (uint32_t)(16 * lane));
        dpre = bc_diagw(pw, r, q);
        dsc = bc_diagw(sw, r, q);
      }
      const int64_t t0 = t0_of(u);
      const int nv = nv_of(t0);
      const auto rgx = rows_rsrc(a.gx + t0 * K, (int64_t)nv * K * 2);
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        // per column c of the lane's 8: grad_phi partial += g^T @ x over the
        // tile's 16 tokens, and grad_x = diag(pre) y + diag(scale) x +
        // (grad_mixes inv) @ phi in one 16x16 accumulator; every MFMA is
        // 16x16x32 (k over tokens x planes for the first three, over m for gs)
        uint32_t o[4][4];
        // four columns at a time, the MFMAs in step order so that four
        // independent accumulations interleave (the gs products first: their
        // operands are ready before the x / grad_y columns are formed)
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          u32x4 xd[4], yd[4];
          floatx4 acc[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            xd[i] = bc_col2(Xr[hh], 4 * k + i);
            yd[i] = bc_col2(grh[hh], 4 * k + i);
          }
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[i] = mfma16x16x32(as_bf16x8(gA0), as_bf16x8(pb[hh][4 * k + i]), floatx4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
          for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)
              ph[hh][mt][4 * k + i] = mfma16x16x32(as_bf16x8(gt[mt]), as_bf16x8(xd[i]), ph[hh][mt][4 * k + i]);
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[i] = mfma16x16x32(as_bf16x8(gA1), as_bf16x8(pb[hh][4 * k + i]), acc[i]);
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[i] = mfma16x16x32(as_bf16x8(dpre), as_bf16x8(yd[i]), acc[i]);
#pragma unroll
          for (int i = 0; i < 4; ++i) acc[i] = mfma16x16x32(as_bf16x8(dsc), as_bf16x8(xd[i]), acc[i]);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            o[e][2 * k] = pack_bf16x2(acc[0][e], acc[1][e]);
            o[e][2 * k + 1] = pack_bf16x2(acc[2][e], acc[3][e]);
          }
        }
        const int colh = slice0 + 128 * hh + 8 * r;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          // rows >= nv fall outside the range and are dropped
          const uint32_t off = (uint32_t)((((4 * q + e) * 4 + n) * D + colh) * 2);
          __builtin_amdgcn_raw_buffer_store_b128(u32x4{o[e][0], o[e][1], o[e][2], o[e][3]}, rgx, off, 0, 2 /* nt */);
        }
      }
      own = own + 1 == G ? 0 : own + 1;
    }
    // ---- (G) the next tile's poll (this wave's buffer is free once it has
    // totalled tile u).  Issued here, after the stores, a load issue that
    // waits for the memory pipeline to take the stores overlaps the wait for
    // tile j below, and the records have had most of an iteration to arrive.
    if (u + 1 >= 0 && u + 1 < nq) issue_poll(u + 1);
    if (j < nq) {
      // ---- (A) tile j landed ---------------------------------------------
      // operations this wave issued after tile j's x loads (iteration j - 1:
      // stores (8), poll (npoll = 4), record words (1), grad_y loads (kg), x
      // loads (8); iteration j: stores (8), poll (4)); away from the steady
      // state all of them
      static_assert(npoll == 4, "the wait below counts four poll loads an iteration");
      if (j >= 3 && j + 2 < nq)
        bc_wait_steady<33>(kg);
      else
        wait_vmcnt<0>();
      // Every wave past this point: tile j's x and grad_y slots landed (each
      // wave's own loads, the grad_y ones issued first), and every wave is
      // done with phase 2 of tile u (its grad_y slot and the shared
      // operands) and with iteration j - 1, so with tile j - 1's x slot
      // (both refilled in (C) below).
      const uint32_t jm3 = (uint32_t)j % 3u;
      bc_sync();
      // ---- (B) phase 1: copy x, grad_pre partial -------------------------
      const uint32_t gslot = bc_opq(gs_l) + (uint32_t)(j & (kBcSg - 1)) * kBcGSlot;
      const uint32_t xslot = bc_opq(xs_l) + jm3 * 32 * 1024 + (uint32_t)(n * 8192 + 16 * lane);
      u32x4 gr1[2][4];
      bc_rd_phase1(Xr, gr1, xslot, gslot + (uint32_t)(16 * lane));
      float pe[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) pe[e] = 0.f;
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) {
        const u32x4 (&gr)[4] = gr1[hh];
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
          for (int w = 0; w < 4; ++w) pe[e] = dot2_bf16(gr[e][w], Xr[hh][e][w], pe[e]);
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) pe[e] = group_sum<15>(pe[e]);  // the 16 lanes of row q: token 4 q + e
      // ---- (D) this wave's words of the record of tile j -------------------
      {
        // word w of chunk c holds values w and w + 8 of the chunk (value v =
        // 4 (token - 4 c) + stream), so the words w = n and n + 4 hold this
        // stream's sums only: lane 16 c + h (row c, whose 16 lanes hold
        // tokens 4 c .. 4 c + 3 in pe[0..3]) stores word n + 4 h of chunk c,
        // tokens 4 c + h and 4 c + h + 2
        const int ck = lane >> 4, h = lane & 1;
        u32x4 word;
        word[0] = __float_as_uint(h ? pe[1] : pe[0]);
        word[1] = __float_as_uint(h ? pe[3] : pe[2]);
        word[2] = word[3] = (uint32_t)(j + 1);
        const uint32_t off =
            (lane & 14) == 0
                ? (uint32_t)(((((j & (kBcR - 1)) * 4 + ck) * G + member) * kBcChunkWords + n + 4 * h) * 16)
                : kBufferOob;
        // default policy: the line stays in this XCC's L2, where the readers' loads find it
        __builtin_amdgcn_raw_buffer_store_b128(word, ring, off, 0, 0);
      }
      // ---- (C) grad_y / per-token data of tile j + 2 into tile u's slot, x
      // of tile j + 2 into the slot of tile j - 1 ------------------------------
      if (j + 2 < nq) issue_g(j + 2);
      if (j + 2 < nq) {
        issue_x(j + 2);
      }
    }
  };

  {
    // two tiles of x in registers: XP holds the even tiles and XQ the odd
    // ones (phase 2 of tile j - 2 and phase 1 of tile j use the same set),
    // so the loop runs two iterations a trip and the ring never moves
    u32x4 XP[2][4], XQ[2][4];
    const int iters = nq + kBcLag;
    for (int j = 0; j < iters; j += 2) {
      step(j, XP);
      if (j + 1 < iters) step(j + 1, XQ);
    }
  }
  wait_vmcnt<0>();  // no direct-to-LDS load may outlive the block

  // ---- this group's grad_phi partial: rows 16 mt + 4 q + v < 24 -----------
#pragma unroll
  for (int hh = 0; hh < 2; ++hh) {
    float* part = a.part + (int64_t)group * M * K + (int64_t)n * D + slice0 + 128 * hh + 8 * r;
#pragma unroll
    for (int mt = 0; mt < 2; ++mt)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int m = 16 * mt + 4 * q + v;
        if (m >= M) continue;
        float4* dst = reinterpret_cast<float4*>(part + (int64_t)m * K);
        dst[0] = float4{ph[hh][mt][0][v], ph[hh][mt][1][v], ph[hh][mt][2][v], ph[hh][mt][3][v]};
        dst[1] = float4{ph[hh][mt][4][v], ph[hh][mt][5][v], ph[hh][mt][6][v], ph[hh][mt][7][v]};
      }
  }
  // ---- grad_alpha[0] / grad_base[0..3] terms of the tiles this member owns
  {
    const float c0 = group_sum<63>(acc_c0);
    const float b = group_sum<60>(acc_b);  // lanes with the same stream m = lane % 4
    if (lane < 4) red[wave][1 + lane] = b;
    if (lane == 0) red[wave][0] = c0;
  }
  __syncthreads();
  if (tid < C) {
    float v = 0.f;
    if (tid == 0 || (tid >= 3 && tid < 7)) {
      const int k = tid == 0 ? 0 : tid - 2;
      v = ((red[0][k] + red[1][k]) + red[2][k]) + red[3][k];
    }
    // row (group, member): the same row holds the same tiles' terms whichever
    // CU the member runs on, so the fixed-order sum is reproducible
    a.contrib[((int64_t)group * G + member) * C + tid] = v;
  }
}

// grad_phi = sum over the groups that formed (read from the control words)
// of their partials, in group order; after a timed-out wait (status word
// nonzero) grad_phi and grad_x become NaN instead.  Block 0 copies the status
// word to the caller's (status_out, may be null; a system-scope store, so it
// may be host memory).
__global__ __launch_bounds__(256) void bc_sum_kernel(const float* __restrict__ part, float* __restrict__ out,
                                                      int64_t n, const uint32_t* ctl, bf16_t* gx, int64_t ngx,
                                                      int32_t* status_out) {
  const uint32_t st = ctl[kCtlStatus];
  const int ng = (int)ctl[kCtlGroups];
  const int64_t i0 = blockIdx.x * (int64_t)blockDim.x + threadIdx.x, stride = (int64_t)gridDim.x * blockDim.x;
  if (blockIdx.x == 0 && threadIdx.x == 0 && status_out)
    __hip_atomic_store(status_out, (int32_t)st, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  if (st) {
    for (int64_t i = i0; i < n; i += stride) out[i] = __builtin_nanf("");
    uint16_t* g = reinterpret_cast<uint16_t*>(gx);
    for (int64_t i = i0; i < ngx; i += stride) g[i] = 0x7FC0u;  // bf16 NaN
    return;
  }
  for (int64_t i = i0; i < n; i += stride) {
    float s = 0.f;
    for (int g = 0; g < ng; ++g) s += part[(int64_t)g * n + i];
    out[i] = s;
  }
}

}  // namespace mhc
