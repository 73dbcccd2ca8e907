// mhc_pre_clamp_sinkhorn forward in one HBM pass over x: N = 4, bf16 x and
// phi, D = 256 G with G = 16 or 28 <= G <= 32 (coop_nch; D = 7168: G = 28).
// Included by pre_fwd.hip.
//
// Semantics: mhc_pre_clamp_sinkhorn_ref, src/mhc_pre_clamp_sinkhorn.py:974-1022;
// with POST also mhc_post_ref before it (src/mhc_post.py:344-352), x_next
// formed in the kernel (the fused post + pre forward).
// The passes it replaces are the reference's RMS / contraction passes over x
// (:897-916) and its y pass (:956), which read x three times.
//
// y needs pre, pre needs the whole N*D row of a token reduced (sum of squares
// and x . phi^T), and a 16-token tile of x is 917 KB at D = 7168: no CU holds
// it.  So G CUs of one XCC form a group that shares every tile: member c owns
// columns [256 c, 256 c + 256) of all four streams (a 32 KB "slice" of a
// 16-token tile) and keeps it in LDS / registers from its one HBM read until
// y of those columns is written.  A block (one per CU) has three kinds of
// waves:
//   L-waves (one per stream) land the slice in an LDS slot by direct-to-LDS
//     loads (one tile ahead, two with x_scaled), contract it with their phi
//     columns on MFMA (16 tokens x 32 m x 256 k) and form the sums of
//     squares; the last of the four adds the four partials in stream order
//     and publishes the member's record (16 tokens x 25 sums) to the group's
//     exchange ring;
//   P-waves (four, tiles taken round robin) total the group's records in two
//     steps once this CU has published a tile: a reduce-scatter (member c
//     reads its share [200 c / G, 200 (c + 1) / G) of the record words from
//     every member, adds them over the members and publishes the totals to
//     the group's totals ring) and a gather (the 40 words y needs, the four
//     pre mixes and the sum of squares of each token, read from their
//     owners' totals); they leave those totals, this member's share and
//     each token's pre / inv_rms (rms_inv / pre_gate, as the finalize
//     kernel) in LDS;
//   Y-waves copy each landed slice into a ring of three tiles of registers
//     (freeing the LDS slot) and, two tiles later, write y (and the optional
//     fp32 x_scaled) of their columns with the P-waves' pre / inv_rms and
//     this member's share of the totals to the [T][M] / [T] buffers that
//     pre_fwd_finalize_kernel turns into mixes, inv_rms, the heads and
//     Sinkhorn afterwards.
// Loads and stores live in different waves (P-waves load and store one
// totals word a lane per tile, Y-waves only store): with loads and stores
// in flight together the compiler waits for the memory counter to reach
// zero wherever one load is needed, which puts a store round trip into
// every tile.  x is read from HBM once; only the 3.2 KB records per member
// and tile and the group's 3.2 KB of totals cross CUs, and they stay in the
// XCC's L2.
//
// Exchange.  A record is 200 16-byte words, each two (value, tag) pairs; the
// tag is the tile's sequence number in its group plus one, so a reader knows
// a value has arrived from its tag alone, with no flags, counters or fences
// (one word is written by one store and read by one load, so it never
// tears); the totals ring uses the same words.  The rings (kCoR tiles per
// group) and the control words are zeroed before every launch.  Records and
// totals are stored with the default policy (the lines stay in the writer's
// XCC L2) and read with device-scope (sc1) loads,
// which skip the reader's CU L1 (it may hold stale copies of the ring) and
// find them in that L2: every member of a group sits on one XCC.
// Membership comes from the XCC_ID hardware register at the start of the
// kernel (a grid-wide registration, so all blocks must be resident: the
// grid is one block per CU and a block's LDS leaves no room for a second on
// its CU, so on a device with no other work every block is resident at
// once), so it holds whichever CU the dispatcher chose for a block.  The
// launch is an ordinary one: a cooperative launch (hipLaunchCooperativeKernel)
// gave the same residency but left the HIP runtime's teardown at process
// exit to crash under rocprofv3.  A block that is not resident in time
// (other work occupying CUs) only delays the others, and their bounded waits
// turn a long delay into a reported failure.
//
// Progress.  L-waves reuse an LDS slot once the Y-waves copied it; P-waves
// reuse their LDS slot once the Y-waves read it; records and totals of
// tile q are overwritten by tile q + kCoR only after every member's P-waves
// are past tile q (kCoR >= 2 S + 2 kCoLag + 2 tiles, see CoCfg: a member
// publishes tile q + kCoR only after its Y-waves used the totals of a later
// tile than q, which every member's P-waves produced after q's).  Every wait is
// bounded: after kCoTimeout of s_memrealtime without progress a wave sets the
// block's abort flag and the status word, and every wave leaves; the finalize
// kernel then writes NaN to every output of the call and copies the status
// word to the caller's status location (mhc_pre_fwd_ex), so the host learns
// of it when the call's work has finished.
#pragma once

#include "coop_common.hpp"

namespace mhc {

constexpr int kCoTT = 16;                          // tokens per tile
constexpr int kCoLW = 4;                           // L-waves: one per stream (N = 4)
constexpr int kCoLag = 2;                          // Y-waves: y of tile j - 2 while tile j lands
constexpr int kCoYW = 4;                           // Y-waves: y writers
constexpr int kCoPW = 4;                           // P-waves: exchange readers
constexpr int kCoPSlots = 4;                       // tiles of P-wave sums in LDS
constexpr int kCoR = 16;                           // exchange ring: tiles per group
constexpr int kCoVals = 25;                        // sums per token: 24 mixes + sum(x^2)
constexpr int kCoRecWords = kCoTT * kCoVals / 2;   // 16-byte words of a record (200)
constexpr int kCoYWords = kCoTT * 5 / 2;           // words y needs: 4 pre mixes + sum(x^2) (40)
constexpr int kCoMaxOW = (kCoRecWords + kCoMinG - 1) / kCoMinG;  // record words a member totals, at most (13)
constexpr int kCoRsB = 16;                         // exchange lanes per member in a load (>= kCoMaxOW)
static_assert(kCoMaxOW <= kCoRsB && kCoMaxG % (kWave / kCoRsB) == 0, "owned words fit a member's lanes");
// forward status codes after the common ones (coop_common.hpp): the wait
// that timed out: 3 L slot copied, 4 L partial buffer, 5 Y tile landed,
// 6 P exchange poll (the members' records), 7 Y sums, 8 P own publish, 9 P
// sums slot, 10 P totals poll (the owners' totals), 11 L x_next formed
// (fused post + pre form)
constexpr uint32_t kStLCopied = 3, kStLPread = 4, kStYLanded = 5, kStPPoll = 6, kStYSums = 7, kStPPub = 8,
                   kStPSlot = 9, kStPTot = 10, kStLXnext = 11;

// Value order inside a record: v * 16 + token, v = 0..3 the pre mixes
// (m = 0..3), v = 4 the sum of squares, v = 5..24 the mixes m = 4..23, so
// the 80 values y needs are the first 40 words.
__host__ __device__ constexpr int co_vidx(int m) { return m < 4 ? m : m + 1; }

template <int NCH>  // 16-byte chunks per stream row of a slice: 16 (128 columns) or 32 (256)
struct CoCfg {
  static_assert(NCH == 16 || NCH == 32, "slice of 128 or 256 columns");
  static constexpr int CS = NCH * 8;                // slice columns
  static constexpr int H = NCH / 16;                // 256-byte half rows per stream row
  static constexpr int STREAM = kCoTT * NCH * 16;   // bytes of one stream of a slot
  static constexpr int SLOT = 4 * STREAM;           // bytes of a slot (one tile slice)
  static constexpr int S = 131072 / SLOT;           // LDS slots: 4 or 8 (128 KB)
  static_assert((S & (S - 1)) == 0, "slot indices are masks");
  // tiles of loads issued ahead: at most S - 2 (the Y-waves may lag one
  // more).  The P-waves' exchange reads share the CU's vector memory path
  // with the direct-to-LDS loads, and with loads two tiles ahead one round
  // of them measured 1.4 - 2.5 us although the records sat in L2.  Without
  // x_scaled one tile ahead measured 3-5% faster than two at the same HBM
  // read rate; with x_scaled's larger stores two stay slightly faster.
  static constexpr int A_MAX = S - 2;
  static constexpr int DMA = STREAM / 1024;         // direct-to-LDS loads per stream and tile
  static constexpr int STEPS = NCH / 4;             // 32-column MFMA steps per stream
  static constexpr int RB = NCH / 4;                // 1 KB row blocks per stream slot (4 tokens x 256 bytes)
  static constexpr int YW = kCoYW;                  // Y-waves
  static constexpr int YB = RB / YW;                // row blocks per Y-wave
  static_assert(YB * YW == RB, "row blocks split evenly over the Y-waves");
  static constexpr int THREADS = (kCoLW + YW + kCoPW) * kWave;
  static_assert(kCoR >= 2 * S + 2 * kCoLag + 2, "exchange ring shorter than the lag it must cover");
  static_assert((kCoR & (kCoR - 1)) == 0 && (kCoPSlots & (kCoPSlots - 1)) == 0, "ring and slot indices are masks");
};

struct CoopArgs {
  PreFwdArgs a;     // inputs and outputs; part / part_ssq receive the designated sums
  uint32_t* ctl;    // kCoCtlWords control words, zeroed before the launch
  u32x4* rec;       // [maxg][kCoR][G][kCoRecWords], zeroed before the launch
  u32x4* tot;       // [maxg][kCoR][kCoRecWords] group totals, zeroed before the launch
  int G;            // members per group (D / CS)
  int maxg;         // groups the ring has room for
  uint64_t timeout; // s_memrealtime ticks a wait may last without progress
  // fused post + pre form (POST): a.x is the post's input x (T, 4, D); the
  // kernel forms x_next = h_res^T x + h_post h_out and writes it once
  const bf16_t* h_out;  // (T, D)
  const float* h_res;   // (T, 4, 4)
  const float* h_post;  // (T, 4)
  bf16_t* x_next;       // (T, 4, D)
};

// The 200 value pairs of a record from the four L-waves' partials (1600
// bytes apart) in one batch: v[it][w] = wave w's pair of word 64 it + lane;
// words 0..191 from a = base + 8 lane, words 192.. from a3 (lanes past the
// record read word 199 again).
__device__ __forceinline__ void co_lds_rd_rec(float2 (&v)[4][4], uint32_t a, uint32_t a3) {
  static_assert(kCoTT * kCoVals * 4 == 1600 && kCoRecWords == 200, "offsets below");
  asm volatile(
      "ds_read_b64 %0, %16\n\t"
      "ds_read_b64 %1, %16 offset:1600\n\t"
      "ds_read_b64 %2, %16 offset:3200\n\t"
      "ds_read_b64 %3, %16 offset:4800\n\t"
      "ds_read_b64 %4, %16 offset:512\n\t"
      "ds_read_b64 %5, %16 offset:2112\n\t"
      "ds_read_b64 %6, %16 offset:3712\n\t"
      "ds_read_b64 %7, %16 offset:5312\n\t"
      "ds_read_b64 %8, %16 offset:1024\n\t"
      "ds_read_b64 %9, %16 offset:2624\n\t"
      "ds_read_b64 %10, %16 offset:4224\n\t"
      "ds_read_b64 %11, %16 offset:5824\n\t"
      "ds_read_b64 %12, %17\n\t"
      "ds_read_b64 %13, %17 offset:1600\n\t"
      "ds_read_b64 %14, %17 offset:3200\n\t"
      "ds_read_b64 %15, %17 offset:4800\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(v[0][0]), "=&v"(v[0][1]), "=&v"(v[0][2]), "=&v"(v[0][3]), "=&v"(v[1][0]), "=&v"(v[1][1]),
        "=&v"(v[1][2]), "=&v"(v[1][3]), "=&v"(v[2][0]), "=&v"(v[2][1]), "=&v"(v[2][2]), "=&v"(v[2][3]),
        "=&v"(v[3][0]), "=&v"(v[3][1]), "=&v"(v[3][2]), "=&v"(v[3][3])
      : "v"(a), "v"(a3)
      : "memory");
}
// eight 16-byte reads at base + o[i]
__device__ __forceinline__ void co_lds_rd8(u32x4 (&v)[8], uint32_t base, const uint32_t (&o)[8]) {
  asm volatile(
      "ds_read_b128 %0, %8\n\t"
      "ds_read_b128 %1, %9\n\t"
      "ds_read_b128 %2, %10\n\t"
      "ds_read_b128 %3, %11\n\t"
      "ds_read_b128 %4, %12\n\t"
      "ds_read_b128 %5, %13\n\t"
      "ds_read_b128 %6, %14\n\t"
      "ds_read_b128 %7, %15\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]), "=&v"(v[6]), "=&v"(v[7])
      : "v"(base + o[0]), "v"(base + o[1]), "v"(base + o[2]), "v"(base + o[3]), "v"(base + o[4]), "v"(base + o[5]),
        "v"(base + o[6]), "v"(base + o[7])
      : "memory");
}
// four 16-byte reads at independent addresses
__device__ __forceinline__ void co_lds_rd4(u32x4 (&v)[4], uint32_t a0, uint32_t a1, uint32_t a2, uint32_t a3) {
  asm volatile(
      "ds_read_b128 %0, %4\n\t"
      "ds_read_b128 %1, %5\n\t"
      "ds_read_b128 %2, %6\n\t"
      "ds_read_b128 %3, %7\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3])
      : "v"(a0), "v"(a1), "v"(a2), "v"(a3)
      : "memory");
}

// h_out's chunk (at a + 32768, the slot's fifth region) and a token's
// h_res row (16 floats at c) and h_post row (4 floats at p) in one batch
__device__ __forceinline__ void co_lds_rd_post(u32x4& h, float (&hr)[16], float (&hp)[4], uint32_t a, uint32_t c,
                                               uint32_t p) {
  u32x4 r[5];
  asm volatile(
      "ds_read_b128 %0, %6 offset:32768\n\t"
      "ds_read_b128 %1, %7\n\t"
      "ds_read_b128 %2, %7 offset:16\n\t"
      "ds_read_b128 %3, %7 offset:32\n\t"
      "ds_read_b128 %4, %7 offset:48\n\t"
      "ds_read_b128 %5, %8\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(h), "=&v"(r[0]), "=&v"(r[1]), "=&v"(r[2]), "=&v"(r[3]), "=&v"(r[4])
      : "v"(a), "v"(c), "v"(p)
      : "memory");
#pragma unroll
  for (int k = 0; k < 4; ++k)
#pragma unroll
    for (int e = 0; e < 4; ++e) hr[4 * k + e] = __uint_as_float(r[k][e]);
#pragma unroll
  for (int e = 0; e < 4; ++e) hp[e] = __uint_as_float(r[4][e]);
}

// x_next of one 16-byte chunk (8 columns) of the four streams: x_next[i] =
// h_post[i] h_out + sum_j h_res[j][i] x[j] in mhc_post's order (the h_post
// product first, then an FMA per input stream in stream order), rounded to
// bf16 (round to nearest even), as the post kernels form it.  In place:
// each word's four inputs are read before its four outputs are written.
__device__ __forceinline__ void co_post_chunk(u32x4 (&X)[4], const u32x4& Hh, const float (&hr)[16],
                                              const float (&hp)[4]) {
#pragma unroll
  for (int wd = 0; wd < 4; ++wd) {
    const float h0 = __uint_as_float(Hh[wd] << 16), h1 = __uint_as_float(Hh[wd] & 0xffff0000u);
    float x0[4], x1[4];
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      x0[jj] = __uint_as_float(X[jj][wd] << 16);
      x1[jj] = __uint_as_float(X[jj][wd] & 0xffff0000u);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v0 = hp[i] * h0, v1 = hp[i] * h1;
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        v0 = fmaf(hr[4 * jj + i], x0[jj], v0);
        v1 = fmaf(hr[4 * jj + i], x1[jj], v1);
      }
      X[i][wd] = pack_bf16x2(v0, v1);
    }
  }
}

// Two 8-byte reads per stream, four streams STRIDE bytes apart: stream n's
// reads at a0 + n STRIDE and a1 + n STRIDE land in v[n][0..1] and v[n][2..3].
template <int STRIDE>
__device__ __forceinline__ void co_lds_rd4x2(u32x4 (&v)[4], uint32_t a0, uint32_t a1) {
  static_assert(3 * STRIDE < 65536, "ds_read offset field");
  u32x2 h[8];
  asm volatile(
      "ds_read_b64 %0, %8\n\t"
      "ds_read_b64 %1, %9\n\t"
      "ds_read_b64 %2, %8 offset:%10\n\t"
      "ds_read_b64 %3, %9 offset:%10\n\t"
      "ds_read_b64 %4, %8 offset:%11\n\t"
      "ds_read_b64 %5, %9 offset:%11\n\t"
      "ds_read_b64 %6, %8 offset:%12\n\t"
      "ds_read_b64 %7, %9 offset:%12\n\t"
      "s_waitcnt lgkmcnt(0)"
      : "=&v"(h[0]), "=&v"(h[1]), "=&v"(h[2]), "=&v"(h[3]), "=&v"(h[4]), "=&v"(h[5]), "=&v"(h[6]), "=&v"(h[7])
      : "v"(a0), "v"(a1), "i"(STRIDE), "i"(2 * STRIDE), "i"(3 * STRIDE)
      : "memory");
#pragma unroll
  for (int n = 0; n < 4; ++n) v[n] = u32x4{h[2 * n][0], h[2 * n][1], h[2 * n + 1][0], h[2 * n + 1][1]};
}

// POST: the fused post + pre forward.  A slot then also holds h_out's slice
// (a fifth 8 KB region, the streams' layout) and the tile's h_res / h_post
// (coefs), so 3 slots of 40 KB fit.  Once a slot has landed, L-wave w and
// Y-wave w form x_next of row blocks w and w + 4 (mhc_post's FMA order and
// rounding) in place; the contraction and the Y-waves' copy wait for all
// eight; the Y-waves write x_next to HBM and keep it for y.
template <int NCH, bool XS, bool POST = false>
__global__ __launch_bounds__(CoCfg<NCH>::THREADS) void pre_fwd_coop_kernel(CoopArgs ca) {
  using C = CoCfg<NCH>;
  static_assert(!(XS && POST), "the fused form writes no x_scaled");
  constexpr int S = POST ? 3 : C::S;                            // LDS slots
  constexpr int SLOT = POST ? C::SLOT + C::STREAM : C::SLOT;     // bytes of a slot
  constexpr int A = POST ? 1 : (XS ? C::A_MAX : 1);
  static_assert(A <= S - 2 && kCoR >= 2 * S + 2 * kCoLag + 2, "slot and ring depths");
  constexpr int H = C::H, DMA = C::DMA, STEPS = C::STEPS, CS = C::CS, YW = C::YW, YB = C::YB;
  constexpr int M = 24;
  constexpr int kCoef = kCoTT * 20;  // floats of a tile's h_res (16 a token) and h_post (4 a token)
  __shared__ __align__(1024) u32x4 slots[S * SLOT / 16];
  __shared__ __align__(16) float coefs[POST ? S : 1][kCoef];
  __shared__ __align__(16) float pbuf[2][kCoLW][kCoTT * kCoVals];   // L-wave partials of a tile (two tiles)
  // per tile: the y words' totals (word w -> [2 w], [2 w + 1]), then this
  // member's owned words' totals
  __shared__ float tot[kCoPSlots][2 * (kCoYWords + kCoMaxOW)];
  __shared__ float pinv[kCoPSlots][kCoTT][5];  // per tile and token: pre (4) and inv_rms
  // counters: landed[S] at 0, copied[S] at 8, pcnt[2] at 16, pread[2] at 18,
  // abort at 21, pub (tiles published) at 22, pready[kCoPSlots] at 24,
  // then ydone[kCoPSlots] and pfinal[kCoPSlots]
  __shared__ uint32_t cnt[24 + 3 * kCoPSlots];
  __shared__ int info[4];

  const PreFwdArgs& a = ca.a;
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t T = a.T;
  const int D = a.D, K = 4 * D, G = ca.G;
  const uint64_t to = ca.timeout;
  uint32_t* status = ca.ctl + kCtlStatus;

  // ---- group formation: the blocks of one XCC, in registration order ------
  if (tid < 24 + 3 * kCoPSlots) cnt[tid] = 0u;
  if (tid == 0) co_register(ca.ctl, G, ca.maxg, ca.timeout, info);
  __syncthreads();
  const int group = info[0], ngroups = info[1], member = info[2];
  if (group < 0) return;  // uniform over the block: not a member of a group
  // tile and loop indices fit 32 bits (the host bounds T); tile sequence qi
  // of this group starts at token t0_of(qi)
  const int ntiles = (int)((T + kCoTT - 1) / kCoTT);
  const int nq = (ntiles - group + ngroups - 1) / ngroups;  // tiles of this group
  if (nq <= 0) return;
  auto t0_of = [&](int qi) { return (int64_t)(group + qi * ngroups) * kCoTT; };
  const int slice0 = member * CS;
  u32x4* recw = ca.rec + (size_t)group * kCoR * G * kCoRecWords;  // this group's ring
  const auto ring = rows_rsrc(recw, (int64_t)kCoR * G * kCoRecWords * 16);
  const uint32_t sbase = lds_addr(slots);
  const uint32_t cbase = lds_addr(&coefs[0][0]);
  // the LDS slot of tile sequence j, and how many tiles used it before j
  auto slot_of = [](int j) -> uint32_t { return (uint32_t)j % (uint32_t)S; };
  auto round_of = [](int j) -> uint32_t { return (uint32_t)j / (uint32_t)S; };
  // (POST: conv[S] at 4, the L-waves' x_next conversions of a slot)
  const uint32_t c_landed = lds_addr(cnt), c_conv = c_landed + 16, c_copied = c_landed + 32, c_pcnt = c_landed + 64,
                 c_pread = c_landed + 72, c_abort = c_landed + 84, c_pub = c_landed + 88, c_pready = c_landed + 96,
                 c_ydone = c_pready + 4 * kCoPSlots, c_pfinal = c_ydone + 4 * kCoPSlots;
  const bf16_t* __restrict__ x = static_cast<const bf16_t*>(a.x);

  if (wave < kCoLW) {
    // ======================= L-wave: stream w ===============================
    const int w = wave, r = lane & 15, q = lane >> 4;
    // phi operands of this stream's slice: step s, m tile mt -> row 16 mt + r,
    // columns w D + slice0 + 32 s + 8 q .. + 8 (zero rows for m >= 24)
    u32x4 B[STEPS][2];
#pragma unroll
    for (int s = 0; s < STEPS; ++s)
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        const int m = 16 * mt + r;
        B[s][mt] = m < M ? ld16(a.phi + (int64_t)m * K + (int64_t)w * D + slice0 + 32 * s + 8 * q) : zero4();
      }
    wait_vmcnt<0>();
    asm volatile("" ::: "memory");

    // direct-to-LDS loads of tile sequence qi, stream w: instruction i moves
    // tokens 4 (i / H) + rho (rho = lane / 16), 256 bytes each; lane rho*16 +
    // kp lands chunk 16 (i % H) + (kp ^ token) of its row (XOR swizzle: the
    // MFMA reads of 16 tokens x one chunk hit 16 different bank groups).
    // Tiles are issued in sequence order, so the tile's first row is a
    // running pointer.  The range ends with the slice of the tile's last
    // token: rows past T (offsets >= nv K 2 > (nv - 1) K 2 + 2 CS) read zeros.
    int iss_t0 = group * kCoTT;  // first token of the next tile issued
    const bf16_t* iss_x = x + ((int64_t)iss_t0 * 4 + w) * D + slice0;
    const int64_t iss_step = (int64_t)ngroups * kCoTT * K;  // elements between a group's tiles
    uint32_t ioff[DMA];
#pragma unroll
    for (int i = 0; i < DMA; ++i) {
      const int tok = 4 * (i / H) + (lane >> 4);
      ioff[i] = (uint32_t)((tok * K + 8 * (16 * (i % H) + ((lane & 15) ^ tok))) * 2);
    }
    // POST: L-wave w also loads instructions 2w, 2w + 1 of h_out's slice
    // (rows of D elements, the streams' layout: tokens 4w + rho, half rows
    // 0 and 1), wave 0 the tile's h_res rows (1 KB) and wave 1 its h_post
    // rows (256 bytes) into the slot's coefs
    static_assert(!POST || (H == 2 && DMA == 8), "h_out's eight loads split two a wave");
    const bf16_t* iss_h = POST ? ca.h_out + (int64_t)iss_t0 * D + slice0 : nullptr;
    uint32_t hoff[2];
#pragma unroll
    for (int ii = 0; ii < 2; ++ii) {
      const int tok = 4 * w + (lane >> 4);
      hoff[ii] = (uint32_t)((tok * D + 8 * (16 * ii + ((lane & 15) ^ tok))) * 2);
    }
    auto issue = [&](int qi) {
      const int64_t left = T - iss_t0;
      const int nv = left < kCoTT ? (int)left : kCoTT;
      const auto rs = rows_rsrc(iss_x, ((int64_t)(nv - 1) * K + CS) * 2);
      const uint32_t sb = sbase + slot_of(qi) * SLOT;
      const uint32_t slot = sb + (uint32_t)(w * C::STREAM);
#pragma unroll
      for (int i = 0; i < DMA; ++i) {
        const uint32_t off = ioff[i];
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void_t*)(uintptr_t)(slot + i * 1024), 16, off, 0, 0,
                                                 2 /* nt */);
      }
      if constexpr (POST) {
        const auto rh = rows_rsrc(iss_h, ((int64_t)(nv - 1) * D + CS) * 2);
        const uint32_t hsl = sb + (uint32_t)(4 * C::STREAM + 2 * w * 1024);
#pragma unroll
        for (int ii = 0; ii < 2; ++ii) {
          const uint32_t off = hoff[ii];
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rh, (lds_void_t*)(uintptr_t)(hsl + ii * 1024), 16, off, 0, 0,
                                                   2 /* nt */);
        }
        const uint32_t cs = cbase + slot_of(qi) * (uint32_t)(kCoef * 4);
        if (w == 0) {
          const auto rr = rows_rsrc(ca.h_res + (int64_t)iss_t0 * 16, (int64_t)nv * 64);
          const uint32_t off = (uint32_t)(lane * 16);
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rr, (lds_void_t*)(uintptr_t)cs, 16, off, 0, 0, 0);
        } else if (w == 1) {
          const auto rp = rows_rsrc(ca.h_post + (int64_t)iss_t0 * 4, (int64_t)nv * 16);
          const uint32_t off = (uint32_t)(lane * 4);
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rp, (lds_void_t*)(uintptr_t)(cs + 1024), 4, off, 0, 0, 0);
        }
        iss_h += (int64_t)ngroups * kCoTT * D;
      }
      iss_t0 += ngroups * kCoTT;
      iss_x += iss_step;
    };
    // LDS address of lane (r, q)'s A operand of step s in a stream slot
    uint32_t aoff[STEPS];
#pragma unroll
    for (int s = 0; s < STEPS; ++s) {
      const int c = 4 * s + q;
      aoff[s] = (uint32_t)((H * (r / 4) + c / 16) * 1024 + (16 * (r % 4) + ((c % 16) ^ r)) * 16);
    }

    for (int j = 0; j < (nq < A ? nq : A); ++j) issue(j);
    for (int j = 0; j < nq; ++j) {
      if (j + A < nq) {
        co_wait_ge(c_copied + 4 * slot_of(j + A), (uint32_t)YW * round_of(j + A), c_abort, status, kStLCopied, to);
        issue(j + A);
      }
      const int after = nq - 1 - j < A ? nq - 1 - j : A;
      if constexpr (POST) {  // loads a tile: 8 + 2, and h_res (wave 0) or h_post (wave 1)
        if (w < 2)
          co_wait_tiles<DMA + 3, A>(after);
        else
          co_wait_tiles<DMA + 2, A>(after);
      } else {
        co_wait_tiles<DMA, A>(after);
      }
      co_lds_inc(c_landed + 4 * slot_of(j));
      if constexpr (POST) {
        // x_next in place of x: once every L-wave's loads of the tile have
        // landed (x of all streams, h_out, the gates), L-wave w converts row
        // block w of the slot (all four streams of those chunks) and Y-wave
        // w row block w + 4; the contraction waits for all eight
        const uint32_t sc = slot_of(j), rc = round_of(j) + 1;
        co_wait_ge(c_landed + 4 * sc, (uint32_t)kCoLW * rc, c_abort, status, kStLXnext, to);
        const uint32_t cs = cbase + sc * (uint32_t)(kCoef * 4);
        {
          const int rb = w;
          const uint32_t o = sbase + sc * SLOT + (uint32_t)(rb * 1024 + lane * 16);
          const uint32_t tk = (uint32_t)(4 * (rb / H) + (lane >> 4));
          u32x4 X[4], Hh;
          float hr[16], hp[4];
          co_lds_rd4(X, o, o + C::STREAM, o + 2 * C::STREAM, o + 3 * C::STREAM);
          co_lds_rd_post(Hh, hr, hp, o, cs + tk * 64u, cs + 1024u + tk * 16u);
          co_post_chunk(X, Hh, hr, hp);
#pragma unroll
          for (int n = 0; n < 4; ++n) co_lds_st4(o + (uint32_t)(n * C::STREAM), __builtin_bit_cast(floatx4, X[n]));
        }
        co_lds_inc(c_conv + 4 * sc);  // after the writes (a wave's LDS operations stay in order)
        co_wait_ge(c_conv + 4 * sc, (uint32_t)(kCoLW + YW) * rc, c_abort, status, kStLXnext, to);
      }

      // contraction of this stream's 16 x CS slice: fresh MFMA chain
      const uint32_t sl = sbase + slot_of(j) * SLOT + (uint32_t)(w * C::STREAM);
      // sum(x^2) on the matrix cores too: the A operand is also the B operand
      // of x x^T (the register layouts coincide), whose diagonal holds each
      // token's sum of squares
      floatx4 acc[2] = {floatx4{0.f, 0.f, 0.f, 0.f}, floatx4{0.f, 0.f, 0.f, 0.f}};
      floatx4 gram = {0.f, 0.f, 0.f, 0.f};
      static_assert(STEPS == 8, "the slice's operands in one batch of eight reads");
      {
        u32x4 Ar[8];
        co_lds_rd8(Ar, sl, aoff);
#pragma unroll
        for (int s = 0; s < STEPS; ++s) {
#pragma unroll
          for (int mt = 0; mt < 2; ++mt) acc[mt] = mfma16x16x32(as_bf16x8(Ar[s]), as_bf16x8(B[s][mt]), acc[mt]);
          gram = mfma16x16x32(as_bf16x8(Ar[s]), as_bf16x8(Ar[s]), gram);
        }
      }
      // token r's sum of squares: row r of column r, element r % 4 of lane (r, r / 4)
      const float g01 = (r & 1) ? gram[1] : gram[0], g23 = (r & 1) ? gram[3] : gram[2];
      const float ssq = (r & 2) ? g23 : g01;

      // partial -> pbuf[j % 2][w]; the buffer's previous tile must be published
      const int pb = j & 1;
      co_wait_ge(c_pread + 4 * (uint32_t)pb, (uint32_t)(j >> 1), c_abort, status, kStLPread, to);
      const uint32_t pw = lds_addr(&pbuf[pb][w][0]);
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        const int m = 16 * mt + r;  // lane (r, q) holds tokens 4q..4q+3 of mix m
        if (m < M) co_lds_st4(pw + (uint32_t)((co_vidx(m) * kCoTT + 4 * q) * 4), acc[mt]);
      }
      if (q == (r >> 2)) co_lds_st(pw + (uint32_t)((4 * kCoTT + r) * 4), ssq);
      // no wait: the count below is raised after these writes (issue order)
      const uint32_t old = co_lds_inc_rtn(c_pcnt + 4 * (uint32_t)pb);
      if (old == 4u * (uint32_t)(j >> 1) + 3u) {
        // last of the four: add the partials in stream order and publish
        const uint32_t tag = (uint32_t)(j + 1);
        // ring layout [tile][member][word]: a record is one contiguous run
        const uint32_t dst = (uint32_t)(((j & (kCoR - 1)) * G + member) * kCoRecWords * 16);  // byte offset in the ring
        const uint32_t p0 = lds_addr(&pbuf[pb][0][0]);
        float2 pr[4][4];
        co_lds_rd_rec(pr, p0 + (uint32_t)(8 * lane),
                      p0 + (uint32_t)(8 * (3 * kWave + (lane < kCoRecWords - 3 * kWave ? lane : kCoRecWords - 1 - 3 * kWave))));
#pragma unroll
        for (int it = 0; it < 4; ++it) {
          const int wd = lane + kWave * it;
          if (wd < kCoRecWords) {
            const float2(&pv)[4] = pr[it];
            u32x4 word;
            word[0] = __float_as_uint(((pv[0].x + pv[1].x) + pv[2].x) + pv[3].x);
            word[1] = tag;
            word[2] = __float_as_uint(((pv[0].y + pv[1].y) + pv[2].y) + pv[3].y);
            word[3] = tag;
            // default policy: the line stays in this XCD's L2, where the
            // readers' device-scope loads find it
            __builtin_amdgcn_raw_buffer_store_b128(word, ring, dst + (uint32_t)(wd * 16), 0, 0);
          }
        }
        co_lds_inc(c_pread + 4 * (uint32_t)pb);
        co_lds_inc(c_pub);
      }
    }
    wait_vmcnt<0>();  // no direct-to-LDS load may outlive the block
    return;
  }

  // The exchange reads and the y stores live in different waves: a wave with
  // both loads and stores in flight gets s_waitcnt vmcnt(0) from the
  // compiler wherever it needs one load (the counter may then decrement out
  // of order), which would put a full store round trip into every tile.
  // P-waves only load (the group's records) and hand sums to the Y-waves
  // through LDS; Y-waves only store (y, x_scaled, part).
  // the record words this member totals for the group: [ow0, ow0 + now)
  const int ow0 = kCoRecWords * member / G;
  const int now = kCoRecWords * (member + 1) / G - ow0;  // <= kCoMaxOW
  // uniform parameters moved to scalar registers up front: a vector register
  // still waiting on its load would make a loop wait on vmcnt(0) (every load
  // or store in flight) at its first use in each iteration
  auto uniform = [](float f) { return __int_as_float(__builtin_amdgcn_readfirstlane(__float_as_int(f))); };
  const float Kf = (float)K;

  if (wave >= kCoLW + YW) {
    // ======================= P-wave pw ======================================
    // P-wave pw takes the tiles u = pw (mod kCoPW) (so kCoPW tiles' polls are
    // in flight at once, and each P-wave owns psum slot pw).  The exchange is
    // a reduce-scatter, then a gather of the words y needs: once this CU has
    // published tile u, (1) it reads its own share [ow0, ow0 + now) of the
    // record words from every member's record, adds them over the members
    // and publishes the totals (same word format and tag) to the group's
    // totals ring; (2) it reads the 40 words y needs from the totals ring
    // (written by their owners) and leaves them, its own share and each
    // token's pre / inv_rms (rms_inv, pre_gate, as the finalize kernel) in
    // LDS for the Y-waves.  A CU so reads 16 bytes per member for each owned
    // word and 640 bytes of totals per tile, instead of 50 words from every
    // member.  Its loads are issued and consumed in the same iteration.
    const int pw = wave - kCoLW - YW;
    static_assert(kCoPSlots == kCoPW, "a psum slot per P-wave");
    const float a0 = uniform(a.alpha[0]);
    float base_n[4];
#pragma unroll
    for (int n = 0; n < 4; ++n) base_n[n] = uniform(a.base[n]);
    // (1) lane l of load q: word ow0 + l % kCoRsB of member q kCoMB + l /
    // kCoRsB.  Tile t's records are a range of exactly G members, so loads
    // of members past G (and lanes past the share) fall outside it and read
    // zeros, whose tag 0 never matches.
    constexpr int kCoMB = kWave / kCoRsB;  // members a load covers (4)
    constexpr int kCoNL = kCoMaxG / kCoMB;  // loads (8)
    const int k1 = lane % kCoRsB;
    const uint32_t roff = k1 < now ? (uint32_t)(((lane / kCoRsB) * kCoRecWords + ow0 + k1) * 16) : kBufferOob;
    auto rec_rsrc = [&](int t) {
      return rows_rsrc(recw + (size_t)(t & (kCoR - 1)) * G * kCoRecWords, (int64_t)G * kCoRecWords * 16);
    };
    u32x4* totw = ca.tot + (size_t)group * kCoR * kCoRecWords;  // this group's totals ring
    auto tot_rsrc = [&](int t) { return rows_rsrc(totw + (size_t)(t & (kCoR - 1)) * kCoRecWords, kCoRecWords * 16); };
    const int sl = pw;
    for (int u = pw; u < nq; u += kCoPW) {
      // this CU's own record comes a few tiles after the previous tile this
      // wave took (a wait of 2 - 3 us measured): fewer, longer sleeps
      co_wait_ge<4>(c_pub, (uint32_t)(u + 1), c_abort, status, kStPPub, to);
      const uint32_t tag = (uint32_t)(u + 1);
      // ---- (1) this member's share from every record, retried until all
      // G now words carry this tile's tag; the sum runs over the loads
      // (members q kCoMB + l / kCoRsB in q order), then over the lanes of the
      // same word (l ^ 16, l ^ 32): a fixed order
      const auto rr = rec_rsrc(u);
      uint64_t deadline = 0;
      float s0 = 0.f, s1 = 0.f;
      for (;;) {
        uint32_t vb = roff;
        asm volatile("" : "+v"(vb));
        u32x4 PV[kCoNL];
#pragma unroll
        for (int q = 0; q < kCoNL; ++q)
          PV[q] = __builtin_amdgcn_raw_buffer_load_b128(rr, vb + (uint32_t)(q * kCoMB * kCoRecWords * 16), 0,
                                                        kCoPolicySc1);
        // a word's two tags are written by one store and read by one load,
        // so they are equal: one is checked
        uint32_t cur = 0;
#pragma unroll
        for (int q = 0; q < kCoNL; ++q) cur += (uint32_t)__popcll(__ballot(PV[q][1] == tag));
        if (cur == (uint32_t)(G * now)) {
          s0 = __uint_as_float(PV[0][0]);
          s1 = __uint_as_float(PV[0][2]);
#pragma unroll
          for (int q = 1; q < kCoNL; ++q) {
            s0 += __uint_as_float(PV[q][0]);
            s1 += __uint_as_float(PV[q][2]);
          }
          s0 = group_sum<48>(s0);
          s1 = group_sum<48>(s1);
          break;
        }
        if (deadline == 0) deadline = co_now() + to;
        if (co_lds_ld_u(c_abort)) break;
        if (co_now() > deadline) {
          co_lds_inc(c_abort);
          co_fail(status, kStPPoll);
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
      // the share's totals to the totals ring (lanes k < now of the first
      // row hold word ow0 + k); default policy: the lines stay in this XCC's
      // L2, where the readers' device-scope loads find them
      const auto tr = tot_rsrc(u);
      if (lane < now)
        __builtin_amdgcn_raw_buffer_store_b128(u32x4{__float_as_uint(s0), tag, __float_as_uint(s1), tag}, tr,
                                               (uint32_t)((ow0 + lane) * 16), 0, 0);
      // ---- (2) the 40 words y needs, from their owners' totals
      deadline = 0;
      float y0 = 0.f, y1 = 0.f;
      for (;;) {
        uint32_t vb = lane < kCoYWords ? (uint32_t)(lane * 16) : kBufferOob;
        asm volatile("" : "+v"(vb));
        const u32x4 TV = __builtin_amdgcn_raw_buffer_load_b128(tr, vb, 0, kCoPolicySc1);
        if (!__any(lane < kCoYWords && TV[1] != tag)) {
          y0 = __uint_as_float(TV[0]);
          y1 = __uint_as_float(TV[2]);
          break;
        }
        if (deadline == 0) deadline = co_now() + to;
        if (co_lds_ld_u(c_abort)) break;
        if (co_now() > deadline) {
          co_lds_inc(c_abort);
          co_fail(status, kStPTot);
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
      // the slot's previous tile must be read by every Y-wave
      co_wait_ge(c_ydone + 4 * (uint32_t)sl, (uint32_t)(YW * (u / kCoPW)), c_abort, status, kStPSlot, to);
      if (lane < kCoYWords) {
        tot[sl][2 * lane] = y0;
        tot[sl][2 * lane + 1] = y1;
      }
      if (lane < now) {
        tot[sl][2 * kCoYWords + 2 * lane] = s0;
        tot[sl][2 * kCoYWords + 2 * lane + 1] = s1;
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      if (lane < kCoTT) {
        const float iv = rms_inv(tot[sl][4 * kCoTT + lane], Kf, a.norm_eps);
#pragma unroll
        for (int n = 0; n < 4; ++n) pinv[sl][lane][n] = pre_gate(tot[sl][n * kCoTT + lane] * iv, a0, base_n[n], a.hc_eps);
        pinv[sl][lane][4] = iv;
      }
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      co_lds_inc(c_pfinal + 4 * (uint32_t)sl);  // after the LDS writes (a wave's LDS operations stay in order)
    }
    return;
  }

  // ========================= Y-wave v =======================================
  // Y-wave v holds row blocks v + YW b (b < YB) of every stream slot: row
  // block rb is tokens 4 (rb / H) + rho (rho = lane / 16), 256-byte half row
  // rb % H; lane rho*16 + kp holds the 16-byte chunk 16 (rb % H) + (kp ^
  // token) of its token (where the direct-to-LDS load put it, so copies are
  // conflict-free 1 KB reads)
  const int v = wave - kCoLW;
  const int rho = lane >> 4, kp = lane & 15;
  int tok[YB], chunk[YB];  // token within a tile and 16-byte chunk of the slice, per row block
#pragma unroll
  for (int b = 0; b < YB; ++b) {
    const int rb = v + YW * b;
    tok[b] = 4 * (rb / H) + rho;
    chunk[b] = 16 * (rb % H) + (kp ^ tok[b]);
  }
  float p[YB][4], inv[YB];  // pre and inv_rms of this lane's tokens
  // With x_scaled the ring and the stores' data fill the register budget:
  // the per-lane addresses are then recomputed from an opaque copy of the
  // lane index at each use instead of being held across the loop (the
  // compiler would spill them, and a scratch reload in this store-only wave
  // waits for every store in flight).
  auto lane_at_use = [&]() -> int {
    int l = lane;
    if constexpr (XS) asm volatile("" : "+v"(l));
    return l;
  };
  auto tok_of = [&](int l, int b) -> int { return 4 * ((v + YW * b) / H) + (l >> 4); };

  // tile j into Xc (POST: x_next; this wave forms row block v + 4 in the
  // slot, the L-waves row blocks 0..3)
  auto copy = [&](int j, u32x4 (&Xc)[YB][4]) {
    co_wait_ge(c_landed + 4 * slot_of(j), (uint32_t)kCoLW * (round_of(j) + 1), c_abort, status, kStYLanded, to);
    if constexpr (POST) {
      static_assert(YB == 2 && 4 * C::STREAM == 32768, "row blocks v and v + 4; h_out at offset 32768");
      const uint32_t sc = slot_of(j);
      const uint32_t o = sbase + sc * SLOT + (uint32_t)((v + YW) * 1024 + lane * 16);
      const uint32_t cs = cbase + sc * (uint32_t)(kCoef * 4);
      int l = lane;  // an opaque lane index: addresses held across the loop would spill
      asm volatile("" : "+v"(l));
      const uint32_t tk = (uint32_t)tok_of(l, 1);
      u32x4 Hh;
      float hr[16], hp[4];
      co_lds_rd4(Xc[1], o, o + C::STREAM, o + 2 * C::STREAM, o + 3 * C::STREAM);
      co_lds_rd_post(Hh, hr, hp, o, cs + tk * 64u, cs + 1024u + tk * 16u);
      co_post_chunk(Xc[1], Hh, hr, hp);
#pragma unroll
      for (int n = 0; n < 4; ++n) co_lds_st4(o + (uint32_t)(n * C::STREAM), __builtin_bit_cast(floatx4, Xc[1][n]));
      co_lds_inc(c_conv + 4 * sc);  // after the writes (a wave's LDS operations stay in order)
      co_wait_ge(c_conv + 4 * sc, (uint32_t)(kCoLW + YW) * (round_of(j) + 1), c_abort, status, kStYLanded, to);
      const uint32_t o0 = sbase + sc * SLOT + (uint32_t)(v * 1024 + lane * 16);
      co_lds_rd4(Xc[0], o0, o0 + C::STREAM, o0 + 2 * C::STREAM, o0 + 3 * C::STREAM);
      co_lds_inc(c_copied + 4 * sc);
      return;
    }
#pragma unroll
    for (int b = 0; b < YB; ++b) {
      if constexpr (XS) {
        // columns 4 kp .. 4 kp + 3 and 64 + 4 kp .. of the half row: chunk
        // kp / 2 and 8 + kp / 2, half kp % 2, each at the lane position
        // chunk ^ token where the direct-to-LDS load put it
        const int l = lane_at_use(), k2 = (l & 15) >> 1, tk = tok_of(l, b);
        const uint32_t o = sbase + slot_of(j) * SLOT + (uint32_t)((v + YW * b) * 1024 + (l >> 4) * 256 + 8 * (l & 1));
        co_lds_rd4x2<C::STREAM>(Xc[b], o + (uint32_t)((k2 ^ tk) * 16), o + (uint32_t)(((8 + k2) ^ tk) * 16));
      } else {
        const uint32_t o = sbase + slot_of(j) * SLOT + (uint32_t)((v + YW * b) * 1024 + lane * 16);
        co_lds_rd4(Xc[b], o, o + C::STREAM, o + 2 * C::STREAM, o + 3 * C::STREAM);
      }
    }
    co_lds_inc(c_copied + 4 * slot_of(j));
  };
  // POST: x_next of tile j's slice to HBM (rows past T fall outside the
  // range and are dropped)
  auto store_xnext = [&](int j, const u32x4 (&Xc)[YB][4]) {
    const int64_t t0 = t0_of(j);
    const int nv = (int)(T - t0 < kCoTT ? T - t0 : kCoTT);
    const auto xn = rows_rsrc(ca.x_next + t0 * 4 * D, (int64_t)nv * 4 * D * 2);
#pragma unroll
    for (int b = 0; b < YB; ++b)
#pragma unroll
      for (int n = 0; n < 4; ++n)
        __builtin_amdgcn_raw_buffer_store_b128(Xc[b][n], xn,
                                               (((uint32_t)tok[b] * 4 + n) * D + (uint32_t)(slice0 + 8 * chunk[b])) * 2,
                                               0, 2 /* nt */);
  };

  // y (and x_scaled) of tile u from Xt with this lane's p / inv: buffer
  // stores against the tile's rows (scalar base, 32-bit offsets; rows past T
  // fall outside the range and are dropped)
  auto write_y = [&](int u, const u32x4 (&Xt)[YB][4]) {
    const int64_t t0 = t0_of(u);
    const int nv = (int)(T - t0 < kCoTT ? T - t0 : kCoTT);
    const auto ys = rows_rsrc(static_cast<bf16_t*>(a.y) + t0 * D, (int64_t)nv * D * 2);
#pragma unroll
    for (int b = 0; b < YB; ++b) {
      float o[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = 0.f;
#pragma unroll
      for (int n = 0; n < 4; ++n)
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          o[2 * w] = fmaf(p[b][n], __uint_as_float(Xt[b][n][w] << 16), o[2 * w]);
          o[2 * w + 1] = fmaf(p[b][n], __uint_as_float(Xt[b][n][w] & 0xffff0000u), o[2 * w + 1]);
        }
      u32x4 ov;
#pragma unroll
      for (int w = 0; w < 4; ++w) ov[w] = pack_bf16x2(o[2 * w], o[2 * w + 1]);
      if constexpr (!XS) {
        const uint32_t col = (uint32_t)(slice0 + 8 * chunk[b]);
        __builtin_amdgcn_raw_buffer_store_b128(ov, ys, ((uint32_t)tok[b] * D + col) * 2, 0, 2 /* nt */);
      } else {
        // columns col0 .. col0 + 3 (registers 0, 1) and col0 + 64 .. (2, 3):
        // every store instruction writes contiguous runs (16-byte pieces at
        // a 32-byte stride, as a lane's 8 columns would give, write at a
        // third of the rate)
        const int l = lane_at_use();
        const uint32_t tk = (uint32_t)tok_of(l, b), col0 = (uint32_t)(slice0 + 128 * ((v + YW * b) % H) + 4 * (l & 15));
        __builtin_amdgcn_raw_buffer_store_b64(u32x2{ov[0], ov[1]}, ys, (tk * D + col0) * 2, 0, 2);
        __builtin_amdgcn_raw_buffer_store_b64(u32x2{ov[2], ov[3]}, ys, (tk * D + col0) * 2 + 128u, 0, 2);
        const auto xr = rows_rsrc(a.x_scaled + t0 * 4 * D, (int64_t)nv * 4 * D * 4);
#pragma unroll
        for (int n = 0; n < 4; ++n)
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            u32x4 xs;
#pragma unroll
            for (int w = 0; w < 2; ++w) {
              const uint32_t xw = Xt[b][n][2 * h + w];
              xs[2 * w] = __float_as_uint(__uint_as_float(xw << 16) * inv[b]);
              xs[2 * w + 1] = __float_as_uint(__uint_as_float(xw & 0xffff0000u) * inv[b]);
            }
            // The stream offset goes into the lane offset, soffset stays the
            // constant 0: with a register soffset the compiler does not
            // separate a 16-byte store from the next write of its data
            // registers, and on gfx950 that lost the data of the last four
            // lanes of each sixteen now and then.
            __builtin_amdgcn_raw_buffer_store_b128(xs, xr, ((tk * 4 + n) * D + col0) * 4 + 256u * h, 0, 2);
          }
      }
    }
  };

  // Step j: copy tile j into X[j % 3], then take tile t = j - 2 from
  // X[t % 3]: pre / inv_rms and this member's share of the totals from the
  // P-waves, y, and (Y-wave 0) the share to part / part_ssq.  The loop body
  // is three steps, so the ring never moves between registers.
  static_assert(kCoLag == 2, "three register buffers: tiles j - 2 .. j");
  auto step = [&](int j, u32x4 (&Xc)[YB][4], const u32x4 (&Xt)[YB][4]) {
    const int t = j - kCoLag;
    if (j < nq) {
      copy(j, Xc);
      if constexpr (POST) store_xnext(j, Xc);
    }
    if (t >= 0 && t < nq) {
      const int sl = t & (kCoPSlots - 1);
      co_wait_ge(c_pfinal + 4 * (uint32_t)sl, (uint32_t)(t / kCoPSlots + 1), c_abort, status, kStYSums, to);
#pragma unroll
      for (int b = 0; b < YB; ++b) {
#pragma unroll
        for (int n = 0; n < 4; ++n) p[b][n] = pinv[sl][tok[b]][n];
        inv[b] = pinv[sl][tok[b]][4];
      }
      // this member's share: record values 2 ow0 .. 2 (ow0 + now) - 1
      // (value vv of token tk for value index 16 vv + tk), from an opaque
      // copy of the lane index (addresses held across the loop would spill)
      int ln = lane;
      asm volatile("" : "+v"(ln));
      const bool hs = v == 0 && ln < 2 * now;
      const float sh = hs ? tot[sl][2 * kCoYWords + ln] : 0.f;
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      co_lds_inc(c_ydone + 4 * (uint32_t)sl);  // slot read
      write_y(t, Xt);
      const int64_t t0 = t0_of(t);
      const int nv = (int)(T - t0 < kCoTT ? T - t0 : kCoTT);
      const int vi = 2 * ow0 + ln, vv = vi / kCoTT, tk = vi % kCoTT;
      // the mixes to part [T][M] (m = vv for vv < 4, vv - 1 past the sum of
      // squares), the sum of squares to part_ssq [T]: two stores, each
      // against one buffer
      if (hs && vv != 4) {
        const auto ps = rows_rsrc(a.part + t0 * M, (int64_t)nv * M * 4);
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(sh), ps, (uint32_t)(tk * M + (vv < 4 ? vv : vv - 1)) * 4,
                                              0, 0);
      }
      if (hs && vv == 4) {
        const auto ss = rows_rsrc(a.part_ssq + t0, (int64_t)nv * 4);
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(sh), ss, (uint32_t)tk * 4, 0, 0);
      }
    }
  };
  u32x4 XA[YB][4], XB[YB][4], XC[YB][4];
  for (int j = 0; j < nq + kCoLag; j += 3) {
    step(j, XA, XB);
    step(j + 1, XB, XC);
    step(j + 2, XC, XA);
  }
}


constexpr int64_t kCoopMinT = 8192;  // below this the split-K forms have lower latency

// Workspace of the single-pass form after kPreFwdWsBase: control words, the
// exchange ring, then part [T][M] and part_ssq [T] (the finalize kernel's
// input) and its pre / inv_rms outputs.  0 if the form does not apply.
inline size_t coop_ws_bytes(int64_t T, int N, int D) {
  int G = 0;
  if (N != 4 || T < kCoopMinT || !coop_nch(D, &G)) return 0;
  return align256((size_t)kCoCtlWords * 4) + align256((size_t)coop_max_groups(G) * kCoR * G * kCoRecWords * 16) +
         align256((size_t)coop_max_groups(G) * kCoR * kCoRecWords * 16) + align256((size_t)T * 24 * 4) +
         align256((size_t)T * 4) + fwd_y_ws_bytes(T, 4);
}

// Runs the single-pass form when it applies (N = 4 bf16 fast path, D with a
// slice geometry, T >= kCoopMinT, enough workspace, not under stream capture,
// a block fits a CU); *used says whether it ran.  The finalize kernel copies
// the status word to a.status_out (when set).
// POST (the fused post + pre forward): `post` carries h_out, h_res, h_post
// and x_next, and a.x is the post's input x.
template <bool XS, bool POST = false>
static int launch_pre_fwd_coop_x(PreFwdArgs a, void* workspace, size_t workspace_bytes, hipStream_t st,
                                  bool* used, const CoopArgs* post = nullptr) {
  *used = false;
  int G = 0;
  const int nch = coop_nch(a.D, &G);
  const size_t need = coop_ws_bytes(a.T, 4, a.D);
  if (!nch || !need || !workspace || workspace_bytes < kPreFwdWsBase + need) return MHC_OK;
  if (stream_capturing(st)) return MHC_OK;
  const void* kfn = (const void*)pre_fwd_coop_kernel<32, XS, POST>;
  const int threads = CoCfg<32>::THREADS;
  if (!coop_fits(kfn, threads, POST ? 2 : 0)) return MHC_OK;
  char* w = static_cast<char*>(workspace) + kPreFwdWsBase;
  CoopArgs ca{};
  if constexpr (POST) {
    ca.h_out = post->h_out;
    ca.h_res = post->h_res;
    ca.h_post = post->h_post;
    ca.x_next = post->x_next;
  }
  ca.ctl = reinterpret_cast<uint32_t*>(w);
  w += align256((size_t)kCoCtlWords * 4);
  ca.rec = reinterpret_cast<u32x4*>(w);
  ca.maxg = coop_max_groups(G);
  ca.timeout = coop_wait_limit();
  const size_t rec_bytes = align256((size_t)ca.maxg * kCoR * G * kCoRecWords * 16);
  w += rec_bytes;
  ca.tot = reinterpret_cast<u32x4*>(w);
  const size_t tot_bytes = align256((size_t)ca.maxg * kCoR * kCoRecWords * 16);
  w += tot_bytes;
  a.part = reinterpret_cast<float*>(w);
  w += align256((size_t)a.T * 24 * 4);
  a.part_ssq = reinterpret_cast<float*>(w);
  w += align256((size_t)a.T * 4);
  a.pre_ws = reinterpret_cast<float*>(w);
  a.inv_ws = reinterpret_cast<float*>(w + align256((size_t)a.T * 4 * 4));
  ca.a = a;
  ca.G = G;
  // zero the control words and the ring (contiguous)
  const int64_t words = (int64_t)((align256((size_t)kCoCtlWords * 4) + rec_bytes + tot_bytes) / 16);
  hipLaunchKernelGGL(co_zero_kernel, dim3(1024), dim3(256), 0, st, reinterpret_cast<u32x4*>(ca.ctl), words);
  int rc = check_launch("pre_fwd_coop_zero");
  if (rc) return rc;
  hipLaunchKernelGGL((pre_fwd_coop_kernel<32, XS, POST>), dim3((unsigned)device_cu_count()), dim3(threads), 0, st, ca);
  if ((rc = check_launch("pre_fwd_coop"))) return rc;
  *used = true;
  a.co_status = ca.ctl + kCtlStatus;  // a timed-out wait turns every output of the call into NaN
  hipLaunchKernelGGL((pre_fwd_finalize_kernel<4>), dim3((unsigned)((a.T + 15) / 16)), dim3(kFwdThreads), 0, st, a, 1);
  return check_launch("pre_fwd_finalize");
}

static int launch_pre_fwd_coop(const PreFwdArgs& a, void* workspace, size_t workspace_bytes, hipStream_t st,
                               bool* used) {
  return a.x_scaled ? launch_pre_fwd_coop_x<true>(a, workspace, workspace_bytes, st, used)
                    : launch_pre_fwd_coop_x<false>(a, workspace, workspace_bytes, st, used);
}

}  // namespace mhc
