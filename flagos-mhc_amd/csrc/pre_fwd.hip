// mhc_pre_clamp_sinkhorn forward, one kernel per call.
//
// Semantics: mhc_pre_clamp_sinkhorn_ref, src/mhc_pre_clamp_sinkhorn.py:974-1022.
//
// A block (4 waves) owns a tile of 64 tokens (4 row blocks of 16):
//   1. contraction  acc[t,m] = sum_k x[t,k] * phi[m,k]  (k = n*D + d) on bf16
//      MFMA 16x16x32: A = 16 tokens x 32 k of x, B = 32 k x 16 m of phi^T.
//      The 4 waves take the 128-column steps of K round-robin, each for all
//      4 row blocks, so a phi operand fetched from L2 serves 64 tokens; the
//      waves' partial sums are reduced through LDS once at the end.  A lane
//      reads 32 consecutive k of its token row (four 16-byte loads streamed
//      past the caches, issued without branches); the four MFMAs of a step
//      consume those groups in the same order for A and B, so the reduction
//      over k is unaffected by the grouping.  The same pass accumulates
//      sum(x^2); mixes = inv_rms * acc, the identity used by the reference's
//      need_backward=False path (src/mhc_pre_clamp_sinkhorn.py:914-916).
//   2. per-token heads and Sinkhorn, one lane per N x N element (sinkhorn.hpp).
//   3. y[t,:] = sum_n pre[t,n] * x[t,n,:], a second pass over the tile's x,
//      and optionally the fp32 x_scaled = x * inv_rms of the reference's
//      need_backward dict.
// fp16 activations / phi are split exactly into two bf16 planes, fp32 ones
// into three; plane products whose indices sum above 2 are dropped, which
// keeps the contraction within ~2^-24 relative of an fp32 dot product.
#include "mhc_launch.hpp"
#include "pre_common.hpp"
#include "pre_host.hpp"
#include "sinkhorn.hpp"

namespace mhc {

constexpr int kFwdTile = 64;  // tokens per block
constexpr size_t kPreFwdWsBase = 256;  // workspace bytes before the split-K area
constexpr int kFwdThreads = 256;

struct PreFwdArgs {
  const void* x;
  const uint16_t* phi;       // bf16 planes [P][M][ld], P <= 3
  int64_t phi_ld;            // row length of a plane (>= K, multiple of 8)
  int64_t phi_plane_stride;  // elements between planes
  int phi_planes;            // 1, 2 or 3
  const float* alpha;
  const float* base;
  float norm_eps, hc_eps, cmin, cmax;
  int apply_clamp;
  int iters;
  void* y;
  float* post_out;
  float* comb;
  float* inv_rms;
  float* mixes;
  float* logits;
  float* pre;
  float* x_scaled;
  int64_t T;
  int D;
  // split-K form (few tiles): contraction stages per split and the partial
  // sums [splits][T][M] / [splits][T], pre / inv_rms of every token for y
  int split_stages;
  float* part;
  float* part_ssq;
  float* pre_ws;
  float* inv_ws;
  // single-pass form: its status word (nonzero when a bounded wait timed
  // out); the finalize kernel then writes NaN to every output of the call
  // and copies the word to status_out (the caller's, may be null)
  const uint32_t* co_status;
  int32_t* status_out;
  // fused post + pre form: x_next (T, N, D) bf16, also set to NaN on failure
  void* x_next_nan;
};

template <int N, typename S, bool VEC, int P>
__global__ __launch_bounds__(kFwdThreads) void pre_fwd_kernel(PreFwdArgs a) {
  using PD = PreDims<N>;
  constexpr int XP = XGroup<S>::PLANES;
  constexpr int M = PD::M, MT = PD::MT, MP = PD::MP;
  constexpr int L = N * N;
  constexpr int RB = kFwdTile / 16;  // 16-token row blocks, all handled by every wave

  __shared__ floatx4 red[4][RB][MT][kWave];
  __shared__ float ssq_sh[4][kFwdTile];
  __shared__ float mix_sh[kFwdTile][MP + 1];
  __shared__ float pre_sh[kFwdTile][N];
  __shared__ float inv_sh[kFwdTile];

  const S* __restrict__ x = static_cast<const S*>(a.x);
  const int D = a.D;
  const int64_t K = (int64_t)N * D;
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, q = lane >> 4;
  const int64_t t0 = (int64_t)blockIdx.x * kFwdTile;

  // row r of each row block; rows past T read row T-1 (and are zeroed)
  const S* xrow[RB];
  bool row_ok[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    const int64_t t = t0 + 16 * rb + r;
    row_ok[rb] = t < a.T;
    xrow[rb] = x + (row_ok[rb] ? t : a.T - 1) * K;
  }
  // phi row 16*mt + r of each plane; rows m >= M read row M-1 (and are zeroed)
  const uint16_t* prow[MT];
  bool m_ok[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = 16 * mt + r;
    m_ok[mt] = m < M;
    prow[mt] = a.phi + (m_ok[mt] ? m : M - 1) * a.phi_ld;
  }

  // ---- 1. contraction + sum of squares ------------------------------------
  // Wave w takes the 128-column steps w, w+4, w+8, ...; lane (r, q) reads
  // columns 32q .. 32q+31 of the step for the 4 row blocks.  phi operands are
  // read from L2 once per step and reused by the 4 row blocks.
  floatx4 acc[RB][MT];
  float ssq[RB];
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
    ssq[rb] = 0.f;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[rb][mt] = floatx4{0.f, 0.f, 0.f, 0.f};
  }
  for (int64_t kb = (int64_t)wave * 128; kb < K; kb += 4 * 128) {
    // MFMA g of the step takes columns kb + 32g + 8q .. +8 on lane (r, q): one load
    // instruction then reads 64 contiguous bytes per row (A and B use the same map)
    const int64_t k = kb + 8 * q;
    u32x4 xp[RB][4][XP];
    // Rows past T read row T-1 and phi rows past M read row M-1: their
    // results land in accumulator rows / columns that are never used, so only
    // the columns of a final partial step (k >= K) need masking.
    const bool full_step = kb + 128 <= K;
    if constexpr (VEC && XP == 1) {
      // bf16: issue all 16 row loads and the phi loads before using any
      u32x4 raw[RB][4];
      if (full_step) {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
          for (int g = 0; g < 4; ++g) raw[rb][g] = ld16nt(xrow[rb] + k + 32 * g);
      } else {
#pragma unroll
        for (int rb = 0; rb < RB; ++rb)
#pragma unroll
          for (int g = 0; g < 4; ++g) raw[rb][g] = ld16_masked(xrow[rb], k + 32 * g, K, true, 2);
      }
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          xp[rb][g][0] = raw[rb][g];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float lo = __uint_as_float(raw[rb][g][i] << 16);
            const float hi = __uint_as_float(raw[rb][g][i] & 0xffff0000u);
            ssq[rb] = fmaf(lo, lo, fmaf(hi, hi, ssq[rb]));
          }
        }
    } else {
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          float f[8];
          XGroup<S>::template load<VEC>(xrow[rb], k + 32 * g, K, row_ok[rb], xp[rb][g], f);
#pragma unroll
          for (int i = 0; i < 8; ++i) ssq[rb] = fmaf(f[i], f[i], ssq[rb]);
        }
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      u32x4 b[P][4];
#pragma unroll
      for (int p = 0; p < P; ++p)
#pragma unroll
        for (int g = 0; g < 4; ++g)
          b[p][g] = full_step ? ld16(prow[mt] + p * a.phi_plane_stride + k + 32 * g)
                              : ld16_masked(prow[mt] + p * a.phi_plane_stride, k + 32 * g, a.phi_ld, true, 2);
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int p = 0; p < P; ++p)
#pragma unroll
          for (int g = 0; g < 4; ++g)
#pragma unroll
            for (int xi = 0; xi < XP; ++xi)
              if (xi + p <= 2)  // dropped cross terms are below 2^-26 relative
                acc[rb][mt] = mfma16x16x32(as_bf16x8(xp[rb][g][xi]), as_bf16x8(b[p][g]), acc[rb][mt]);
    }
  }

  // ---- cross-wave reduction -------------------------------------------------
  // acc layout: lane (r, q) holds D[i = 4q + v][j = r]: token 16*rb + 4q + v, m = 16*mt + r
#pragma unroll
  for (int rb = 0; rb < RB; ++rb) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) red[wave][rb][mt][lane] = acc[rb][mt];
    float s = ssq[rb];
    s += __shfl_xor(s, 16, kWave);
    s += __shfl_xor(s, 32, kWave);
    if (q == 0) ssq_sh[wave][16 * rb + r] = s;
  }
  __syncthreads();
  for (int idx = tid; idx < kFwdTile * MP; idx += kFwdThreads) {
    const int tt = idx / MP, m = idx - (idx / MP) * MP;
    const int rb = tt >> 4, i = tt & 15;
    const int mt = m >> 4, ln = (m & 15) + 16 * (i >> 2), v = i & 3;
    const float sacc = red[0][rb][mt][ln][v] + red[1][rb][mt][ln][v] + red[2][rb][mt][ln][v] +
                       red[3][rb][mt][ln][v];
    const float ss = ssq_sh[0][tt] + ssq_sh[1][tt] + ssq_sh[2][tt] + ssq_sh[3][tt];
    const float inv = 1.0f / sqrtf(ss / (float)K + a.norm_eps);
    mix_sh[tt][m] = sacc * inv;
    if (m == 0) inv_sh[tt] = inv;
  }
  __syncthreads();

  if (a.mixes) {
    for (int idx = tid; idx < kFwdTile * M; idx += kFwdThreads) {
      const int tt = idx / M, m = idx - (idx / M) * M;
      if (t0 + tt < a.T) a.mixes[(t0 + tt) * M + m] = mix_sh[tt][m];
    }
  }
  if (a.inv_rms && tid < kFwdTile && t0 + tid < a.T) a.inv_rms[t0 + tid] = inv_sh[tid];

  // ---- 2. heads + Sinkhorn, lane per matrix element -----------------------
  {
    constexpr int TPP = kFwdThreads / L;  // tokens per pass
    constexpr int PASSES = kFwdTile / TPP;
    const float a0 = a.alpha[0], a1 = a.alpha[1], a2 = a.alpha[2];
    for (int ps = 0; ps < PASSES; ++ps) {
      const int tt = ps * TPP + tid / L;
      const int e = tid % L;
      const int64_t tok = t0 + tt;
      const bool ok = tok < a.T;
      const float logit = mix_sh[tt][2 * N + e] * a2 + a.base[2 * N + e];
      const float lc = clamp_logit(logit, a.apply_clamp, a.cmin, a.cmax);
      const float c = sinkhorn_fwd<N>(lc, a.hc_eps, a.iters);
      if (ok) {
        a.comb[tok * L + e] = c;
        if (a.logits) a.logits[tok * L + e] = logit;
      }
      if (e < N) {
        const float p = sigmoidf_(mix_sh[tt][e] * a0 + a.base[e]) + a.hc_eps;
        pre_sh[tt][e] = p;
        if (ok && a.pre) a.pre[tok * N + e] = p;
      } else if (e < 2 * N) {
        const float po = 2.0f * sigmoidf_(mix_sh[tt][e] * a1 + a.base[e]);
        if (ok) a.post_out[tok * N + (e - N)] = po;
      }
    }
  }
  __syncthreads();

  // ---- 3. y = sum_n pre[n] * x[n] (+ x_scaled) ---------------------------
  // Each thread takes YU units (8 columns of one token) per round and issues
  // all their loads before using any, so enough bytes are in flight.
  S* __restrict__ y = static_cast<S*>(a.y);
  constexpr int YU = 4;
  const int DG = (D + 7) / 8;
  int64_t ntok = a.T - t0;
  if (ntok > kFwdTile) ntok = kFwdTile;
  const int units = (int)ntok * DG;
  for (int u0 = tid; u0 < units; u0 += YU * kFwdThreads) {
    float f[YU][N][8];
#pragma unroll
    for (int j = 0; j < YU; ++j) {
      const int u = u0 + j * kFwdThreads;
      const int tt = u / DG, dg = u - (u / DG) * DG;
      const bool ok = u < units;
#pragma unroll
      for (int n = 0; n < N; ++n)
        load8f<S, VEC>(x + ((t0 + (ok ? tt : 0)) * N + n) * D, (int64_t)dg * 8, D, ok, f[j][n]);
    }
#pragma unroll
    for (int j = 0; j < YU; ++j) {
      const int u = u0 + j * kFwdThreads;
      if (u >= units) break;
      const int tt = u / DG, dg = u - (u / DG) * DG;
      const int64_t tok = t0 + tt, d = (int64_t)dg * 8;
      float o[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = 0.f;
#pragma unroll
      for (int n = 0; n < N; ++n) {
        const float p = pre_sh[tt][n];
#pragma unroll
        for (int i = 0; i < 8; ++i) o[i] = fmaf(p, f[j][n][i], o[i]);
      }
      store8<S, VEC>(y + tok * D, d, D, o);
      if (a.x_scaled) {
        const float inv = inv_sh[tt];
#pragma unroll
        for (int n = 0; n < N; ++n) {
          float xs[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) xs[i] = f[j][n][i] * inv;
          store8<float, VEC>(a.x_scaled + tok * K + (int64_t)n * D, d, D, xs);
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// LDS-pipelined form: N = 4 or 8, bf16 x and phi (phi used in place),
// D % 8 == 0, 16-byte aligned rows.
//
// A persistent block per CU walks its 64-token tiles; every tile is a stream
// of contraction stages through one ring of S stage slots in LDS, filled by
// direct-to-LDS loads issued S-1 stages ahead (no registers held by loads
// in flight): 128 columns of K each, x[64 tokens][128] (16 KB) and
// phi[32 rows][128] (8 KB, rows >= M zero).  Wave w multiplies row block w
// (tokens 16w..16w+15) by all of phi: no cross-wave reduction.  A load
// instruction moves 4 rows x 256 contiguous bytes.  In a slot a row is 256
// bytes with its 16-byte chunks XOR-swizzled by (row & 15), so the MFMA
// operand reads (16 rows, one chunk each) hit 16 different chunk positions:
// conflict-free.  After the last contraction stage the wave's accumulators
// give mixes; heads and Sinkhorn run as in the generic kernel while the next
// tile's first stages are already loading, and pre / inv_rms go to the
// workspace for the y kernel (pre_fwd_y_kernel, a block per token), which
// reads x a second time.  The y pass used to run as stages of this kernel
// (4 tokens x 512 columns each); as its own block-per-token kernel it moves
// its 4.7 GB (N = 4, D = 7168, T = 65536) in 0.78 ms instead of sharing the
// ring (pre forward 1.57 -> 1.44 ms on one MI355X).
// ---------------------------------------------------------------------------

// 16-byte LDS read, complete when the statement ends (see lds_read4).
__device__ __forceinline__ u32x4 pre_sh4(uint32_t a) {
  u32x4 v;
  asm volatile("ds_read_b128 %0, %1\n\ts_waitcnt lgkmcnt(0)" : "=v"(v) : "v"(a) : "memory");
  return v;
}
// Slot geometry per N: 16 units of x and 4*MT of phi (MT 16-row m blocks);
// 1 KB units.
// N = 4: two blocks per CU, each with a 3-slot ring (2 x 79 KB of LDS),
// measured 2% faster than one block with 4 slots; N = 8 fits one block.
// N = 8 (80 phi rows, 36 KB slots, one block per CU): heads and Sinkhorn of
// a 64-token tile take 16 passes of 4 tokens (a wave per 8 x 8 token), which
// stalled the block's ring for a third of its time (contraction 400 -> 254
// us without them at D = 2048, T = 32768).  N = 8 therefore writes each
// tile's sums to the workspace and the split form's token-parallel finalize
// kernel runs heads and Sinkhorn over all tokens; without the mixes buffer a
// fourth ring slot fits.  This kernel runs N = 8 only in its split form: the
// persistent N = 8 contraction is pre_fwd_ks8_kernel below.
template <int N> struct FwdDmaCfg {
  static constexpr int MT = PreDims<N>::MT;
  static constexpr int UNITS = 16 + 4 * MT;
  static constexpr bool HEADS_APART = N != 4;
  static constexpr int S = HEADS_APART ? 4 : 3;      // slots (LDS: S * UNITS KB [+ mixes])
  static constexpr int BLOCKS_PER_CU = N == 4 ? 2 : 1;
};

// SPLIT: block (tile, s) runs contraction stages [s * split_stages, ..) of
// one tile and writes its partial sums; heads and y run in two more kernels.
// Otherwise a persistent block runs all stages of its tiles and the heads.
template <int N, bool SPLIT>
__global__ __launch_bounds__(kFwdThreads) void pre_fwd_dma_kernel(PreFwdArgs a) {
  using C = FwdDmaCfg<N>;
  constexpr int M = PreDims<N>::M, MT = C::MT, L = N * N, TT = kFwdTile, S = C::S, UNITS = C::UNITS;
  constexpr int CW = 128;                  // K columns per contraction stage
  constexpr int CI = 4 + MT;               // loads per wave and stage
  // Stage j's loads have landed once at most VM_C newer vector memory
  // operations are outstanding: the loads of the S - 2 stages issued after
  // it.  The heads' stores after a tile's last stage only add newer
  // operations, so the same bound then waits a little longer than needed.
  constexpr int VM_C = (S - 2) * CI;
  static_assert(N % 4 == 0 && VM_C < 64, "vmcnt range");
  __shared__ u32x4 ring[S * UNITS * kWave];
  __shared__ float mix_sh[C::HEADS_APART ? 1 : TT][M + 1];
  __shared__ __align__(16) float inv_sh[TT];

  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, q = lane >> 4;
  const int D = a.D;
  const int K = N * D;
  const int64_t T = a.T;
  const int nst_c = (K + CW - 1) / CW;
  const int64_t ntiles = (T + TT - 1) / TT;
  // stage range of this block within its tiles: [s_first, per_tile)
  const int s_first = SPLIT ? (int)blockIdx.y * a.split_stages : 0;
  const int per_tile = SPLIT ? (s_first + a.split_stages < nst_c ? s_first + a.split_stages : nst_c) : nst_c;
  const int64_t my_tiles = SPLIT ? (blockIdx.x < ntiles ? 1 : 0)
                                 : (ntiles - blockIdx.x + gridDim.x - 1) / gridDim.x;
  if (my_tiles <= 0 || s_first >= per_tile) return;  // uniform over the block
  const int64_t J = my_tiles * (per_tile - s_first);
  const bf16_t* __restrict__ x = static_cast<const bf16_t*>(a.x);
  const auto rphi = rows_rsrc(a.phi, (int64_t)M * K * 2);

  // per-thread constants of the heads / Sinkhorn step
  const int e = tid % L;
  const float a0 = a.alpha[0], a1 = a.alpha[1], a2 = a.alpha[2];
  const float base_l = a.base[2 * N + e];
  const float base_h = e < 2 * N ? a.base[e] : 0.f;

  // ---- loads of stage j --------------------------------------------------
  int64_t itile = blockIdx.x;  // tile and stage of the next issue
  int is = s_first;
  auto issue = [&](int64_t j) {
    const int64_t tb = itile * TT;
    const int nv = (int)(T - tb < TT ? T - tb : TT);
    const uint32_t slot = lds_addr(ring) + (uint32_t)((j % S) * UNITS * 1024);
    const auto rx = rows_rsrc(x + tb * K, (int64_t)nv * K * 2);
    const int k0 = is * CW;
    // units 0..15: x rows 4u..4u+3 (u = wave + 4i, i < 4); 16..: phi rows
    // 4(u-16)..+3 (u = 16 + wave + 4(i-4)); chunks XOR-swizzled by row & 15
#pragma unroll
    for (int i = 0; i < CI; ++i) {
      const int u = wave + 4 * i;
      const int row = 4 * (wave + 4 * (i < 4 ? i : i - 4)) + q;
      const int k = k0 + 8 * (r ^ (row & 15));
      const uint32_t off = k < K ? (uint32_t)(((int64_t)row * K + k) * 2) : kBufferOob;
      lds_void_t* dst = (lds_void_t*)(uintptr_t)(slot + u * 1024);
      if (i < 4)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, dst, 16, off, 0, 0, 2 /* nt */);
      else
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rphi, dst, 16, off, 0, 0, 0);
    }
    if (++is == per_tile) {
      is = s_first;
      itile += gridDim.x;
    }
  };

  for (int64_t j = 0; j < S - 1 && j < J; ++j) issue(j);

  floatx4 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = floatx4{0.f, 0.f, 0.f, 0.f};
  float ssq = 0.f;
  int64_t ctile = blockIdx.x;
  int cs = s_first;  // stage of the current tile being consumed
  for (int64_t j = 0; j < J; ++j) {
    // this wave's loads of stage j have landed (see VM_C); near the end
    // fewer stages follow it and everything is waited for
    if (j + S - 2 < J)
      wait_vmcnt<VM_C>();
    else
      wait_vmcnt<0>();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    const uint32_t slot = lds_addr(ring) + (uint32_t)((j % S) * UNITS * 1024);
    const int64_t tb = ctile * TT;

    // ---- contraction stage: row block `wave` x all of phi ----------------
    if (j + S - 1 < J) issue(j + S - 1);
    // chunk 4g+q of x row 16*wave + r and of phi rows 16*mt + r: the
    // swizzled positions differ per g, so each read has its own address;
    // phi row 16*mt + r sits mt*4 KB after row r
    u32x4 A[4], B[MT][4];
    const uint32_t ca = slot + (16 * wave + r) * 256, cb0 = slot + 16 * 1024 + r * 256;
    uint32_t sw[4];
#pragma unroll
    for (int g = 0; g < 4; ++g) sw[g] = ((4 * g + q) ^ r) << 4;
    if constexpr (MT == 2) {
      asm volatile(
          "ds_read_b128 %0, %12\n\t"
          "ds_read_b128 %1, %13\n\t"
          "ds_read_b128 %2, %14\n\t"
          "ds_read_b128 %3, %15\n\t"
          "ds_read_b128 %4, %16\n\t"
          "ds_read_b128 %5, %17\n\t"
          "ds_read_b128 %6, %18\n\t"
          "ds_read_b128 %7, %19\n\t"
          "ds_read_b128 %8, %16 offset:4096\n\t"
          "ds_read_b128 %9, %17 offset:4096\n\t"
          "ds_read_b128 %10, %18 offset:4096\n\t"
          "ds_read_b128 %11, %19 offset:4096\n\t"
          "s_waitcnt lgkmcnt(0)"
          : "=&v"(A[0]), "=&v"(A[1]), "=&v"(A[2]), "=&v"(A[3]), "=&v"(B[0][0]), "=&v"(B[0][1]),
            "=&v"(B[0][2]), "=&v"(B[0][3]), "=&v"(B[1][0]), "=&v"(B[1][1]), "=&v"(B[1][2]), "=&v"(B[1][3])
          : "v"(ca + sw[0]), "v"(ca + sw[1]), "v"(ca + sw[2]), "v"(ca + sw[3]), "v"(cb0 + sw[0]),
            "v"(cb0 + sw[1]), "v"(cb0 + sw[2]), "v"(cb0 + sw[3])
          : "memory");
    } else {
      // N = 8: phi rows 32..79 as well, all 24 reads before one wait (one
      // wave per SIMD: the LDS latency is paid once a stage)
      static_assert(MT == 5, "phi row blocks read here");
      asm volatile(
          "ds_read_b128 %0, %24\n\t"
          "ds_read_b128 %1, %25\n\t"
          "ds_read_b128 %2, %26\n\t"
          "ds_read_b128 %3, %27\n\t"
          "ds_read_b128 %4, %28\n\t"
          "ds_read_b128 %5, %29\n\t"
          "ds_read_b128 %6, %30\n\t"
          "ds_read_b128 %7, %31\n\t"
          "ds_read_b128 %8, %28 offset:4096\n\t"
          "ds_read_b128 %9, %29 offset:4096\n\t"
          "ds_read_b128 %10, %30 offset:4096\n\t"
          "ds_read_b128 %11, %31 offset:4096\n\t"
          "ds_read_b128 %12, %28 offset:8192\n\t"
          "ds_read_b128 %13, %29 offset:8192\n\t"
          "ds_read_b128 %14, %30 offset:8192\n\t"
          "ds_read_b128 %15, %31 offset:8192\n\t"
          "ds_read_b128 %16, %28 offset:12288\n\t"
          "ds_read_b128 %17, %29 offset:12288\n\t"
          "ds_read_b128 %18, %30 offset:12288\n\t"
          "ds_read_b128 %19, %31 offset:12288\n\t"
          "ds_read_b128 %20, %28 offset:16384\n\t"
          "ds_read_b128 %21, %29 offset:16384\n\t"
          "ds_read_b128 %22, %30 offset:16384\n\t"
          "ds_read_b128 %23, %31 offset:16384\n\t"
          "s_waitcnt lgkmcnt(0)"
          : "=&v"(A[0]), "=&v"(A[1]), "=&v"(A[2]), "=&v"(A[3]), "=&v"(B[0][0]), "=&v"(B[0][1]),
            "=&v"(B[0][2]), "=&v"(B[0][3]), "=&v"(B[1][0]), "=&v"(B[1][1]), "=&v"(B[1][2]), "=&v"(B[1][3]),
            "=&v"(B[2][0]), "=&v"(B[2][1]), "=&v"(B[2][2]), "=&v"(B[2][3]), "=&v"(B[3][0]), "=&v"(B[3][1]),
            "=&v"(B[3][2]), "=&v"(B[3][3]), "=&v"(B[4][0]), "=&v"(B[4][1]), "=&v"(B[4][2]), "=&v"(B[4][3])
          : "v"(ca + sw[0]), "v"(ca + sw[1]), "v"(ca + sw[2]), "v"(ca + sw[3]), "v"(cb0 + sw[0]),
            "v"(cb0 + sw[1]), "v"(cb0 + sw[2]), "v"(cb0 + sw[3])
          : "memory");
    }
    // The stage's 128 columns go through a fresh 4-step MFMA chain that is
    // then added to the running sums with round-to-nearest-even adds: a
    // single MFMA accumulator chain over all of K (up to ~900 steps) drifts
    // measurably (2e-5 relative at K = 16384).
    floatx4 part[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) part[mt] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int g = 0; g < 4; ++g) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float lo = __uint_as_float(A[g][i] << 16), hi = __uint_as_float(A[g][i] & 0xffff0000u);
        ssq = fmaf(lo, lo, fmaf(hi, hi, ssq));
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) part[mt] = mfma16x16x32(as_bf16x8(A[g]), as_bf16x8(B[mt][g]), part[mt]);
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] += part[mt];

    if ((SPLIT || C::HEADS_APART) && cs == per_tile - 1) {
      // ---- this split's partial sums of the tile (or, persistent with
      // HEADS_APART, the tile's sums: blockIdx.y = 0) ----------------------
      // acc: lane (r, q) holds token 16*wave + 4q + v, m = 16*mt + r; after
      // the shuffles the lanes of row r hold this split's sum(x^2) of token
      // 16*wave + r
      ssq += __shfl_xor(ssq, 16, kWave);
      ssq += __shfl_xor(ssq, 32, kWave);
      const int64_t pbase = (int64_t)blockIdx.y * T;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int64_t tok = tb + 16 * wave + 4 * q + v;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          if (tok < T && 16 * mt + r < M) a.part[(pbase + tok) * M + 16 * mt + r] = acc[mt][v];
      }
      if (q == 0 && tb + 16 * wave + r < T) a.part_ssq[pbase + tb + 16 * wave + r] = ssq;
      if constexpr (!SPLIT) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[mt] = floatx4{0.f, 0.f, 0.f, 0.f};
        ssq = 0.f;
      }
    } else if (!SPLIT && !C::HEADS_APART && cs == nst_c - 1) {
      // ---- tile's mixes, heads and Sinkhorn -----------------------------
      // acc: lane (r, q) holds token 16*wave + 4q + v, m = 16*mt + r; the
      // lane of row r (any q) holds sum(x^2) of token 16*wave + r
      ssq += __shfl_xor(ssq, 16, kWave);
      ssq += __shfl_xor(ssq, 32, kWave);
      const float inv_row = 1.0f / sqrtf(ssq / (float)K + a.norm_eps);
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float inv = __shfl(inv_row, 4 * q + v, kWave);
        const int tt = 16 * wave + 4 * q + v;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
          if (16 * mt + r < M) mix_sh[tt][16 * mt + r] = acc[mt][v] * inv;
      }
      if (q == 0) inv_sh[16 * wave + r] = inv_row;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) acc[mt] = floatx4{0.f, 0.f, 0.f, 0.f};
      ssq = 0.f;
      __syncthreads();
      if (a.mixes) {
        for (int idx = tid; idx < TT * M; idx += kFwdThreads) {
          const int tt = idx / M, m = idx - (idx / M) * M;
          if (tb + tt < T) a.mixes[(tb + tt) * M + m] = mix_sh[tt][m];
        }
      }
      if (tid < TT && tb + tid < T) {
        a.inv_ws[tb + tid] = inv_sh[tid];
        if (a.inv_rms) a.inv_rms[tb + tid] = inv_sh[tid];
      }
      constexpr int TPP = kFwdThreads / L;
#pragma unroll 1
      for (int ps = 0; ps < TT / TPP; ++ps) {
        const int tt = ps * TPP + tid / L;
        const int64_t tok = tb + tt;
        const bool ok = tok < T;
        const float logit = mix_sh[tt][2 * N + e] * a2 + base_l;
        const float lc = clamp_logit(logit, a.apply_clamp, a.cmin, a.cmax);
        const float c = sinkhorn_fwd<N>(lc, a.hc_eps, a.iters);
        if (ok) {
          a.comb[tok * L + e] = c;
          if (a.logits) a.logits[tok * L + e] = logit;
        }
        if (e < N) {
          const float p = sigmoidf_(mix_sh[tt][e] * a0 + base_h) + a.hc_eps;
          if (ok) {
            a.pre_ws[tok * N + e] = p;
            if (a.pre) a.pre[tok * N + e] = p;
          }
        } else if (e < 2 * N) {
          const float po = 2.0f * sigmoidf_(mix_sh[tt][e] * a1 + base_h);
          if (ok) a.post_out[tok * N + (e - N)] = po;
        }
      }
      __syncthreads();
    }
    if (++cs == per_tile) {
      cs = s_first;
      ctile += gridDim.x;
    }
  }
}

// ---------------------------------------------------------------------------
// N = 8 persistent contraction with the K steps split over waves.
//
// A tile of TT tokens streams through a ring of S slots in LDS, one slot per
// stage of CW columns of K: x[TT][CW] and phi[80][CW], filled by direct-to-LDS
// loads S - 1 stages ahead, one block of 8 waves (two per SIMD) per CU.  Wave
// (g, kq) takes 32 tokens (two 16-row blocks) and k-step kq (32 columns) of
// every stage against all 80 phi rows: it reads 7 KB of a slot (the 4-wave
// kernel read all of phi for each of 4 row blocks, 24 KB a wave), and one
// wave's waits overlap the other's MFMA and VALU work.  A 1 KB unit holds
// 1024 / (2 CW) rows; row R keeps its chunk c (8 columns) at position
// c ^ f(R), f(R) = R & 15 for CW = 128 and (R >> 1) & 7 for CW = 64, so the
// 16 rows of an MFMA operand read hit 16 different 16-byte bank groups.
// Each wave runs a fresh 4-step MFMA chain over 4 stages that is then added
// to its running sums (one chain over all of K drifts); at a tile's last
// stage the k-step waves hand their sums to the kq = 0 waves in a fixed
// order through the just-read slot, and those write the tile's sums to the
// workspace for the finalize kernel (heads, Sinkhorn).
//   TT = 64, CW = 128 (S = 4, 36 KB slots): 48 KB of x in flight per CU.
//   TT = 128, CW = 64 (S = 5, 26 KB slots): 64 KB of x in flight and half
//   the phi bytes per x byte; used when every CU gets a 128-token tile.
// ---------------------------------------------------------------------------
constexpr int kKsWaves = 8;
constexpr int kKsThreads = kKsWaves * kWave;

template <int TT, int CW> struct KsCfg {
  static constexpr int M = PreDims<8>::M, MT = PreDims<8>::MT;
  static constexpr int RB = TT / 16, KS = CW / 32;           // row blocks, k-steps per stage
  static constexpr int NG = kKsWaves / KS;                   // row-block pairs
  static constexpr int CPR = CW / 8;                         // 16-byte chunks per row
  static constexpr int RPU = 1024 / (2 * CW);                // rows per 1 KB unit
  static constexpr int XU = TT / RPU, PU = M / RPU;          // x and phi units of a slot
  static constexpr int UNITS = XU + PU;
  static constexpr int S = CW == 128 ? 4 : 5;  // 6 slots of 26 KB measured no faster than 5
  static_assert(RB == 2 * NG && M % RPU == 0 && XU % kKsWaves == 0, "two row blocks a wave, whole units");
  static_assert(S * UNITS <= 144, "ring within the LDS");
  __device__ static constexpr int swz(int row) { return CW == 128 ? (row & 15) : ((row >> 1) & 7); }
};

template <int TT, int CW>
__global__ __launch_bounds__(kKsThreads) void pre_fwd_ks8_kernel(PreFwdArgs a) {
  constexpr int N = 8;
  using C = KsCfg<TT, CW>;
  constexpr int M = C::M, MT = C::MT, S = C::S, UNITS = C::UNITS, KS = C::KS;
  constexpr int CIMAX = (UNITS + kKsWaves - 1) / kKsWaves;
  constexpr int CIMIN = UNITS / kKsWaves;
  constexpr int XI = C::XU / kKsWaves;  // the first XI loads of a wave are x units
  // Stage j's loads have landed once at most VM_C newer vector memory
  // operations are outstanding: the loads of the S - 2 stages issued after it
  // (at least CIMIN a wave each); the tile sums' stores only add newer ones.
  constexpr int VM_C = (S - 2) * CIMIN;
  static_assert(VM_C < 64 && MT == 5, "vmcnt range; five phi row blocks read below");
  static_assert(2 * 2 * MT * kWave * 16 + 2 * 2 * 16 * 4 <= UNITS * 1024, "hand-over of two waves fits a slot");
  __shared__ u32x4 ring[S * UNITS * kWave];

  const int lane = threadIdx.x & (kWave - 1);
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int kq = wv % KS, g = wv / KS;
  const int r = lane & 15, q = lane >> 4;
  const int D = a.D;
  const int K = N * D;
  const int64_t T = a.T;
  const int nst_c = (K + CW - 1) / CW;
  const int64_t ntiles = (T + TT - 1) / TT;
  const int64_t my_tiles = (ntiles - blockIdx.x + gridDim.x - 1) / gridDim.x;
  if (my_tiles <= 0) return;  // uniform over the block
  const int64_t J = my_tiles * nst_c;
  const bf16_t* __restrict__ x = static_cast<const bf16_t*>(a.x);
  const auto rphi = rows_rsrc(a.phi, (int64_t)M * K * 2);
  const int nci = wv < UNITS - CIMIN * kKsWaves ? CIMAX : CIMIN;

  // ---- loads of stage j: unit u = wv + 8i (x units first, then phi);
  // DMA lane L: row RPU * unit + L / CPR, position L % CPR
  const int lrow = lane / C::CPR, lpos = lane % C::CPR;
  int64_t itile = blockIdx.x;
  int is = 0;
  auto issue = [&](int64_t j) {
    const int64_t tb = itile * TT;
    const int nv = (int)(T - tb < TT ? T - tb : TT);
    const uint32_t slot = lds_addr(ring) + (uint32_t)((j % S) * UNITS * 1024);
    const auto rx = rows_rsrc(x + tb * K, (int64_t)nv * K * 2);
    const int k0 = is * CW;
#pragma unroll
    for (int i = 0; i < CIMAX; ++i) {
      if (i < nci) {
        const int u = wv + kKsWaves * i;
        const int row = C::RPU * (i < XI ? u : u - C::XU) + lrow;
        const int k = k0 + 8 * (lpos ^ C::swz(row));
        const uint32_t off = k < K ? (uint32_t)(((int64_t)row * K + k) * 2) : kBufferOob;
        lds_void_t* dst = (lds_void_t*)(uintptr_t)(slot + u * 1024);
        if (i < XI)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, dst, 16, off, 0, 0, 2 /* nt */);
        else
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rphi, dst, 16, off, 0, 0, 0);
      }
    }
    if (++is == nst_c) {
      is = 0;
      itile += gridDim.x;
    }
  };

  for (int64_t j = 0; j < S - 1 && j < J; ++j) issue(j);

  floatx4 acc[2][MT], part[2][MT];
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[b][mt] = part[b][mt] = floatx4{0.f, 0.f, 0.f, 0.f};
  float ssq[2] = {0.f, 0.f};
  // chunk KS... : lane (r, q) reads chunk 4kq + q of rows with row & 15 = r
  // (rows 32g + 16b + r of x, 16mt + r of phi: f depends on r only)
  const uint32_t roff = (uint32_t)(r * 2 * CW + ((4 * kq + q) ^ C::swz(r)) * 16);
  int64_t ctile = blockIdx.x;
  int cs = 0;  // stage of the current tile
  for (int64_t j = 0; j < J; ++j) {
    if (j + S - 2 < J)
      wait_vmcnt<VM_C>();
    else
      wait_vmcnt<0>();
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    const uint32_t slot = lds_addr(ring) + (uint32_t)((j % S) * UNITS * 1024);
    // the next loads go to the slot of stage j - 1, which every wave finished
    // reading before the barrier
    if (j + S - 1 < J) issue(j + S - 1);

    // x rows 32g + r and 32g + 16 + r, phi rows 16mt + r: chunk 4kq + q
    u32x4 A[2], B[MT];
    asm volatile(
        "ds_read_b128 %0, %7\n\t"
        "ds_read_b128 %1, %7 offset:%9\n\t"
        "ds_read_b128 %2, %8\n\t"
        "ds_read_b128 %3, %8 offset:%9\n\t"
        "ds_read_b128 %4, %8 offset:%10\n\t"
        "ds_read_b128 %5, %8 offset:%11\n\t"
        "ds_read_b128 %6, %8 offset:%12\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(A[0]), "=&v"(A[1]), "=&v"(B[0]), "=&v"(B[1]), "=&v"(B[2]), "=&v"(B[3]), "=&v"(B[4])
        : "v"(slot + 32 * g * 2 * CW + roff), "v"(slot + C::XU * 1024 + roff), "i"(16 * 2 * CW),
          "i"(32 * 2 * CW), "i"(48 * 2 * CW), "i"(64 * 2 * CW)
        : "memory");
    if ((cs & 3) == 0) {
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) part[b][mt] = floatx4{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int b = 0; b < 2; ++b) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float lo = __uint_as_float(A[b][i] << 16), hi = __uint_as_float(A[b][i] & 0xffff0000u);
        ssq[b] = fmaf(lo, lo, fmaf(hi, hi, ssq[b]));
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) part[b][mt] = mfma16x16x32(as_bf16x8(A[b]), as_bf16x8(B[mt]), part[b][mt]);
    }
    const bool last = cs == nst_c - 1;
    if ((cs & 3) == 3 || last) {
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[b][mt] += part[b][mt];
    }

    if (last) {
      // ---- the tile's sums: lane (r, q) of acc[b][mt] holds token
      // 32g + 16b + 4q + v, m = 16mt + r; after the shuffles the lanes of row
      // r hold this wave's sum(x^2) of token 32g + 16b + r.  The k-step
      // waves kq = 1.. hand theirs to wave kq = 0 of their pair in turn, two
      // waves a round, through this stage's slot: [pair slot][b][mt][lane]
      // floatx4, then ssq [pair slot][b][r].
#pragma unroll
      for (int b = 0; b < 2; ++b) {
        ssq[b] += __shfl_xor(ssq[b], 16, kWave);
        ssq[b] += __shfl_xor(ssq[b], 32, kWave);
      }
      floatx4* xch = reinterpret_cast<floatx4*>(ring + (size_t)(j % S) * UNITS * kWave);
      float* xss = reinterpret_cast<float*>(xch + 2 * 2 * MT * kWave);
#pragma unroll 1
      for (int k = 1; k < KS; ++k) {
#pragma unroll 1
        for (int g0 = 0; g0 < C::NG; g0 += 2) {
          const bool mine = g >= g0 && g < g0 + 2;
          const int ps = g - g0;  // pair slot of this round
          __syncthreads();        // the slot's operands or the previous hand-over have been read
          if (mine && kq == k) {
#pragma unroll
            for (int b = 0; b < 2; ++b) {
#pragma unroll
              for (int mt = 0; mt < MT; ++mt) xch[((ps * 2 + b) * MT + mt) * kWave + lane] = acc[b][mt];
              if (q == 0) xss[(ps * 2 + b) * 16 + r] = ssq[b];
            }
          }
          __syncthreads();
          if (mine && kq == 0) {
#pragma unroll
            for (int b = 0; b < 2; ++b) {
#pragma unroll
              for (int mt = 0; mt < MT; ++mt) acc[b][mt] += xch[((ps * 2 + b) * MT + mt) * kWave + lane];
              ssq[b] += xss[(ps * 2 + b) * 16 + r];
            }
          }
        }
      }
      if (kq == 0) {
        const int64_t tb = ctile * TT;
#pragma unroll
        for (int b = 0; b < 2; ++b) {
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            const int64_t tok = tb + 32 * g + 16 * b + 4 * q + v;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
              if (tok < T) a.part[tok * M + 16 * mt + r] = acc[b][mt][v];
          }
          const int64_t tok = tb + 32 * g + 16 * b + r;
          if (q == 0 && tok < T) a.part_ssq[tok] = ssq[b];
        }
      }
#pragma unroll
      for (int b = 0; b < 2; ++b) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[b][mt] = floatx4{0.f, 0.f, 0.f, 0.f};
        ssq[b] = 0.f;
      }
      __syncthreads();  // the hand-over has been read before the slot is loaded again
    }
    if (++cs == nst_c) {
      cs = 0;
      ctile += gridDim.x;
    }
  }
}

// ---- split-K form, kernels 2 and 3 -----------------------------------------
// Kernel 2: one N x N lane group per token sums the splits' partials in split
// order, then computes inv_rms, mixes, heads, clamp and Sinkhorn exactly as
// the single-kernel form does after its last contraction stage.
template <int N>
__global__ __launch_bounds__(kFwdThreads) void pre_fwd_finalize_kernel(PreFwdArgs a, int nsplit) {
  constexpr int M = PreDims<N>::M, L = N * N, TPP = kFwdThreads / L;
  const int tid = threadIdx.x, e = tid % L;
  const int64_t T = a.T;
  const int64_t tok = (int64_t)blockIdx.x * TPP + tid / L;
  const bool ok = tok < T;
  const int64_t tk = ok ? tok : T - 1;  // lanes past T compute on the last token and store nothing
  const float K = (float)(N * a.D);
  float ssq = 0.f, acc_l = 0.f, acc_h = 0.f;
  // unconditional loads (lanes e >= 2N sum a column they never use), so the
  // unrolled iterations issue together instead of waiting one by one
  const int eh = e < 2 * N ? e : 0;
#pragma unroll 8
  for (int s = 0; s < nsplit; ++s) {
    const int64_t row = (int64_t)s * T + tk;
    ssq += a.part_ssq[row];
    acc_l += a.part[row * M + 2 * N + e];
    acc_h += a.part[row * M + eh];
  }
  // a failed single-pass run makes every output of the call NaN (y and
  // x_scaled rows included) rather than leave wrong values behind
  const uint32_t co_st = a.co_status ? *a.co_status : 0u;
  const bool failed = co_st != 0u;
  // the caller's status word, which may live in host memory: a system-scope
  // store writes through to it
  if (a.co_status && a.status_out && blockIdx.x == 0 && tid == 0)
    __hip_atomic_store(a.status_out, (int32_t)co_st, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  const float inv = failed ? __builtin_nanf("") : rms_inv(ssq, K, a.norm_eps);
  const float mix_l = acc_l * inv, mix_h = acc_h * inv;
  if (failed) {
    const int64_t t0 = (int64_t)blockIdx.x * TPP;
    const int64_t nt = T - t0 < TPP ? T - t0 : TPP;
    uint16_t* y = static_cast<uint16_t*>(a.y);  // the single-pass form's y is bf16
    for (int64_t i = tid; i < nt * a.D; i += kFwdThreads) y[t0 * a.D + i] = 0x7FC0u;  // bf16 NaN
    if (a.x_scaled)
      for (int64_t i = tid; i < nt * N * a.D; i += kFwdThreads) a.x_scaled[t0 * N * a.D + i] = __builtin_nanf("");
    if (a.x_next_nan) {
      uint16_t* xn = static_cast<uint16_t*>(a.x_next_nan);
      for (int64_t i = tid; i < nt * N * a.D; i += kFwdThreads) xn[t0 * N * a.D + i] = 0x7FC0u;
    }
  }
  if (ok) {
    if (a.mixes) {
      a.mixes[tok * M + 2 * N + e] = mix_l;
      if (e < 2 * N) a.mixes[tok * M + e] = mix_h;
    }
    if (e == 0) {
      a.inv_ws[tok] = inv;
      if (a.inv_rms) a.inv_rms[tok] = inv;
    }
  }
  const float a0 = a.alpha[0], a1 = a.alpha[1], a2 = a.alpha[2];
  const float logit = mix_l * a2 + a.base[2 * N + e];
  const float lc = clamp_logit(logit, a.apply_clamp, a.cmin, a.cmax);
  // (the clamp would turn a NaN logit into a bound: NaN is set directly)
  const float c = failed ? __builtin_nanf("") : sinkhorn_fwd<N>(lc, a.hc_eps, a.iters);
  if (ok) {
    a.comb[tok * L + e] = c;
    if (a.logits) a.logits[tok * L + e] = logit;
  }
  if (e < N) {
    const float p = pre_gate(mix_h, a0, a.base[e], a.hc_eps);
    if (ok) {
      a.pre_ws[tok * N + e] = p;
      if (a.pre) a.pre[tok * N + e] = p;
    }
  } else if (e < 2 * N) {
    const float po = 2.0f * sigmoidf_(mix_h * a1 + a.base[e]);
    if (ok) a.post_out[tok * N + (e - N)] = po;
  }
}

// y[t, d] = sum_n pre[t, n] * x[t, n, d] (and x_scaled = x * inv_rms): a
// block per token of W = min(16, ceil(D / 512)) waves, wave w taking the
// 512-column chunks w, w + W, .. (8 columns a lane), so a token's rows are read
// as a few long contiguous streams (the order that lets the post kernels
// move mixed traffic fastest); x is read once here (non-temporal), y and
// x_scaled are written once (streaming stores).  Same FMA order as the
// generic kernel's y.
constexpr int kFwdYWaves = 16;

template <int N, bool XS>
__global__ __launch_bounds__(kWave * kFwdYWaves) void pre_fwd_y_kernel(PreFwdArgs a) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), W = blockDim.x / kWave;
  const int64_t t = blockIdx.x;
  const int D = a.D;
  float p[N];
#pragma unroll
  for (int n = 0; n < N; ++n) p[n] = a.pre_ws[t * N + n];
  if constexpr (XS) {
    // lane l takes columns 4 l .. 4 l + 3 and 256 + 4 l .. of each chunk, so
    // every store instruction writes one contiguous run (fp32 16-byte pieces
    // at a 32-byte lane stride, as 8 columns a lane would give, write at
    // about a third of the contiguous rate).  D % 8 == 0: a 4-column piece
    // is in range when its first column is.
    const float inv = a.inv_ws[t];
    for (int c0 = wave * 512; c0 < D; c0 += W * 512) {
      const int col = c0 + 4 * lane;
      const bool hi = col + 256 < D;  // the lane's second piece is in range
      const bf16_t* x = static_cast<const bf16_t*>(a.x) + t * N * D + col;
      u32x2 X[2][N];  // all loads before any store (one in-order counter covers both)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int n = 0; n < N; ++n)
          X[h][n] = (h == 0 ? col < D : hi)
                        ? __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(x + (int64_t)n * D + 256 * h))
                        : u32x2{0u, 0u};
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        if (!(h == 0 ? col < D : hi)) break;
        float o[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int n = 0; n < N; ++n)
#pragma unroll
          for (int w = 0; w < 2; ++w) {
            o[2 * w] = fmaf(p[n], __uint_as_float(X[h][n][w] << 16), o[2 * w]);
            o[2 * w + 1] = fmaf(p[n], __uint_as_float(X[h][n][w] & 0xffff0000u), o[2 * w + 1]);
          }
        const u32x2 ov = {pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
        __builtin_nontemporal_store(ov,
                                    reinterpret_cast<u32x2*>(static_cast<bf16_t*>(a.y) + t * D + col + 256 * h));
#pragma unroll
        for (int n = 0; n < N; ++n) {
          u32x4 xs;
#pragma unroll
          for (int w = 0; w < 2; ++w) {
            xs[2 * w] = __float_as_uint(__uint_as_float(X[h][n][w] << 16) * inv);
            xs[2 * w + 1] = __float_as_uint(__uint_as_float(X[h][n][w] & 0xffff0000u) * inv);
          }
          st16nt(a.x_scaled + (t * N + n) * (int64_t)D + col + 256 * h, xs);
        }
      }
    }
    return;
  }
  for (int col = wave * 512 + 8 * lane; col < D; col += W * 512) {
    const bf16_t* x = static_cast<const bf16_t*>(a.x) + t * N * D + col;
    u32x4 X[N];
#pragma unroll
    for (int n = 0; n < N; ++n) X[n] = ld16nt(x + (int64_t)n * D);
    float o[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = 0.f;
#pragma unroll
    for (int n = 0; n < N; ++n)
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        o[2 * w] = fmaf(p[n], __uint_as_float(X[n][w] << 16), o[2 * w]);
        o[2 * w + 1] = fmaf(p[n], __uint_as_float(X[n][w] & 0xffff0000u), o[2 * w + 1]);
      }
    u32x4 ov;
#pragma unroll
    for (int w = 0; w < 4; ++w) ov[w] = pack_bf16x2(o[2 * w], o[2 * w + 1]);
    st16nt(static_cast<bf16_t*>(a.y) + t * D + col, ov);
  }
}

template <int N>
static int launch_pre_fwd_y(const PreFwdArgs& a, hipStream_t st) {
  const int chunks = (a.D + 511) / 512;
  const int waves = chunks < kFwdYWaves ? chunks : kFwdYWaves;
  const dim3 grid((unsigned)a.T), block(kWave * waves);
  // Blocks of 12 or more waves run one token per CU at a time (D = 6144 /
  // 7168: 1.5% / 2% faster); narrower ones faster several to a CU (D = 4096:
  // 267 -> 247 us for the operator at T = 16384; D = 5120: 2%).
  const size_t lds = waves >= 12 ? one_block_per_cu_lds() : 0;
  if (int rc = check_grid(grid, block, "mhc_pre_fwd")) return rc;
  if (a.x_scaled)
    hipLaunchKernelGGL((pre_fwd_y_kernel<N, true>), grid, block, lds, st, a);
  else
    hipLaunchKernelGGL((pre_fwd_y_kernel<N, false>), grid, block, lds, st, a);
  return check_launch("pre_fwd_y");
}

int launch_pre_y_pass(const void* x, const float* pre, void* y, int64_t T, int N, int D, hipStream_t st) {
  PreFwdArgs a{};
  a.x = x;
  a.pre_ws = const_cast<float*>(pre);
  a.y = y;
  a.T = T;
  a.D = D;
  if (N == 4) return launch_pre_fwd_y<4>(a, st);
  if (N == 8) return launch_pre_fwd_y<8>(a, st);
  return set_error(MHC_ERR_UNSUPPORTED, "pre y pass: N=%d not supported (4, 8)", N);
}

struct FwdSplitPlan {
  int nsplit = 0, stages = 0;
  size_t bytes = 0;  // workspace for partials, pre and inv_rms
};


// Workspace of the persistent form when heads run in the finalize kernel
// (N = 8): the tiles' sums [T][M] and sum(x^2) [T], then pre and inv_rms.
static size_t heads_apart_bytes(int64_t T, int N) {
  if (N == 4 || T <= 0) return 0;
  const int M = 2 * N + N * N;
  return align256((size_t)T * M * 4) + align256((size_t)T * 4) + fwd_y_ws_bytes(T, N);
}

static FwdSplitPlan fwd_split_plan(int64_t T, int N, int D) {
  FwdSplitPlan p;
  const int64_t ntiles = (T + kFwdTile - 1) / kFwdTile;
  const int nst_c = (int)(((int64_t)N * D + 127) / 128);
  if (T <= 0 || ntiles > 256) return p;
  int64_t want = (512 + ntiles - 1) / ntiles;
  if (want > nst_c / 4) want = nst_c / 4;
  if (want > 64) want = 64;
  if (want < 2) return p;
  p.stages = (int)((nst_c + want - 1) / want);
  p.nsplit = (nst_c + p.stages - 1) / p.stages;
  const int M = 2 * N + N * N;
  p.bytes = align256((size_t)p.nsplit * T * M * 4) + align256((size_t)p.nsplit * T * 4) +
            align256((size_t)T * N * 4) + align256((size_t)T * 4);
  return p;
}

}  // namespace mhc

#include "pre_fwd_coop.hpp"

namespace mhc {

// The LDS-pipelined kernel covers the bf16 fast path (N = 4, 8).  Buffer
// ranges are 32-bit: a tile of x rows (64 * N * D, fp32 x_scaled) must fit.
static bool fwd_dma_usable(const PreFwdArgs& a, int N, bool bf16x, bool vec) {
  return (N == 4 || N == 8) && bf16x && vec && a.phi_planes == 1 && a.phi_ld == (int64_t)N * a.D &&
         (int64_t)kFwdTile * N * a.D * 4 < ((int64_t)1 << 31) && aligned16(a.phi);
}

template <int N>
static int launch_pre_fwd_dma(PreFwdArgs a, void* workspace, size_t workspace_bytes, hipStream_t st) {
  if constexpr (N == 4) {  // x read from HBM once where the single-pass form applies
    bool used = false;
    const int rc = launch_pre_fwd_coop(a, workspace, workspace_bytes, st, &used);
    if (rc || used) return rc;
  }
  const int64_t ntiles = (a.T + kFwdTile - 1) / kFwdTile;
  const FwdSplitPlan plan = fwd_split_plan(a.T, N, a.D);
  if (plan.nsplit >= 2 && workspace && workspace_bytes >= kPreFwdWsBase + plan.bytes) {
    // few tiles: split K over blocks, then heads and y in their own kernels
    char* w = static_cast<char*>(workspace) + kPreFwdWsBase;
    const int M = 2 * N + N * N;
    a.split_stages = plan.stages;
    a.part = reinterpret_cast<float*>(w);
    w += align256((size_t)plan.nsplit * a.T * M * 4);
    a.part_ssq = reinterpret_cast<float*>(w);
    w += align256((size_t)plan.nsplit * a.T * 4);
    a.pre_ws = reinterpret_cast<float*>(w);
    w += align256((size_t)a.T * N * 4);
    a.inv_ws = reinterpret_cast<float*>(w);
    hipLaunchKernelGGL((pre_fwd_dma_kernel<N, true>), dim3((unsigned)ntiles, (unsigned)plan.nsplit),
                       dim3(kFwdThreads), 0, st, a);
    int rc = check_launch("pre_fwd_split");
    if (rc) return rc;
    constexpr int TPP = kFwdThreads / (N * N);
    hipLaunchKernelGGL((pre_fwd_finalize_kernel<N>), dim3((unsigned)((a.T + TPP - 1) / TPP)), dim3(kFwdThreads),
                       0, st, a, plan.nsplit);
    if ((rc = check_launch("pre_fwd_finalize"))) return rc;
    return launch_pre_fwd_y<N>(a, st);
  }
  // contraction and heads in one persistent kernel (N = 8: contraction, then
  // heads in the finalize kernel), then y
  char* w = static_cast<char*>(workspace) + kPreFwdWsBase;
  if constexpr (FwdDmaCfg<N>::HEADS_APART) {  // the caller checked heads_apart_bytes
    const int M = 2 * N + N * N;
    a.part = reinterpret_cast<float*>(w);
    w += align256((size_t)a.T * M * 4);
    a.part_ssq = reinterpret_cast<float*>(w);
    w += align256((size_t)a.T * 4);
  }
  a.pre_ws = reinterpret_cast<float*>(w);
  a.inv_ws = reinterpret_cast<float*>(w + align256((size_t)a.T * N * 4));
  const int64_t cus = device_cu_count();
  const int64_t slots = cus * FwdDmaCfg<N>::BLOCKS_PER_CU;  // resident blocks (LDS rings)
  const int64_t grid = ntiles < slots ? ntiles : slots;
  if constexpr (N == 8) {
    // 128-token tiles once they fill every CU, else 64-token tiles
    const int64_t nt128 = (a.T + 127) / 128;
    if (nt128 >= cus)
      hipLaunchKernelGGL((pre_fwd_ks8_kernel<128, 64>), dim3((unsigned)cus), dim3(kKsThreads), 0, st, a);
    else
      hipLaunchKernelGGL((pre_fwd_ks8_kernel<64, 128>), dim3((unsigned)grid), dim3(kKsThreads), 0, st, a);
  } else
    hipLaunchKernelGGL((pre_fwd_dma_kernel<N, false>), dim3((unsigned)grid), dim3(kFwdThreads), 0, st, a);
  int rc = check_launch("pre_fwd_dma");
  if (rc) return rc;
  if constexpr (FwdDmaCfg<N>::HEADS_APART) {
    constexpr int TPP = kFwdThreads / (N * N);
    hipLaunchKernelGGL((pre_fwd_finalize_kernel<N>), dim3((unsigned)((a.T + TPP - 1) / TPP)), dim3(kFwdThreads),
                       0, st, a, 1);
    if ((rc = check_launch("pre_fwd_finalize"))) return rc;
  }
  return launch_pre_fwd_y<N>(a, st);
}

template <int N, typename S, int P>
static int launch_pre_fwd_p(const PreFwdArgs& a, bool vec, hipStream_t st) {
  const dim3 grid((unsigned)((a.T + kFwdTile - 1) / kFwdTile)), block(kFwdThreads);
  if (vec)
    hipLaunchKernelGGL((pre_fwd_kernel<N, S, true, P>), grid, block, 0, st, a);
  else
    hipLaunchKernelGGL((pre_fwd_kernel<N, S, false, P>), grid, block, 0, st, a);
  return check_launch("pre_fwd");
}

template <int N, typename S>
static int launch_pre_fwd(const PreFwdArgs& a, bool vec, hipStream_t st) {
  switch (a.phi_planes) {
    case 1: return launch_pre_fwd_p<N, S, 1>(a, vec, st);
    case 2: return launch_pre_fwd_p<N, S, 2>(a, vec, st);
    case 3: return launch_pre_fwd_p<N, S, 3>(a, vec, st);
  }
  return set_error(MHC_ERR_INVALID, "mhc_pre_fwd: %d phi planes", a.phi_planes);
}

template <typename S>
static int dispatch_pre_fwd(int N, const PreFwdArgs& a, bool vec, hipStream_t st) {
  switch (N) {
    case 4: return launch_pre_fwd<4, S>(a, vec, st);
    case 8: return launch_pre_fwd<8, S>(a, vec, st);
  }
  return set_error(MHC_ERR_UNSUPPORTED, "mhc_pre_fwd: N=%d not supported (4, 8)", N);
}

}  // namespace mhc

using namespace mhc;

// Workspace of the two-pass forms (every path runs with this much).
static size_t pre_fwd_ws_min(int64_t T, int32_t N, int32_t D, int32_t phi_dtype) {
  if (N <= 0 || D <= 0) return 0;
  const int M = 2 * N + N * N;
  const int64_t K = (int64_t)N * D;
  if (phi_dtype == MHC_DTYPE_BF16 && K % 8 == 0) {  // phi used directly: pre / inv_rms for the y
    const size_t split = fwd_split_plan(T, N, D).bytes;  // kernel, split-K partials for few tiles
    size_t y = fwd_y_ws_bytes(T < 0 ? 0 : T, N);
    const size_t ha = heads_apart_bytes(T, N);           // N = 8: tile sums for the finalize kernel
    if (ha > y) y = ha;
    return kPreFwdWsBase + (split > y ? split : y);
  }
  return align256(phi_planes_bytes(phi_dtype, M, K));
}

// With room for the single-pass form where it applies (N = 4, bf16 phi).
extern "C" size_t mhc_pre_fwd_workspace_size(int64_t T, int32_t N, int32_t D, int32_t phi_dtype) {
  const size_t base = pre_fwd_ws_min(T, N, D, phi_dtype);
  if (phi_dtype != MHC_DTYPE_BF16) return base;
  const size_t coop = coop_ws_bytes(T, N, D);
  return coop && kPreFwdWsBase + coop > base ? kPreFwdWsBase + coop : base;
}

// Whether mhc_pre_fwd / mhc_pre_fwd_ex without x_scaled runs the single-pass
// form on these arguments (the checks launch_pre_fwd_dma<4> and
// launch_pre_fwd_coop make, in the same order).  The fused post + pre
// forward defers to the two operators where it does.
namespace mhc {
bool pre_fwd_single_pass_applies(const void* x, int32_t x_dtype, const void* phi, int32_t phi_dtype, const void* y,
                                 size_t workspace_bytes, int64_t T, int32_t N, int32_t D, hipStream_t st) {
  if (N != 4 || x_dtype != MHC_DTYPE_BF16 || phi_dtype != MHC_DTYPE_BF16 || D <= 0 || T <= 0) return false;
  const int64_t K = (int64_t)N * D;
  if (K % 8 || !aligned16(phi) || D % 8 || !aligned16(x) || !aligned16(y)) return false;
  if ((int64_t)kFwdTile * N * D * 4 >= ((int64_t)1 << 31)) return false;
  const size_t y_ws = fwd_y_ws_bytes(T, N), ha_ws = heads_apart_bytes(T, N);
  if (workspace_bytes < kPreFwdWsBase + (ha_ws > y_ws ? ha_ws : y_ws)) return false;
  int G = 0;
  const size_t need = coop_ws_bytes(T, 4, D);
  if (!coop_nch(D, &G) || !need || workspace_bytes < kPreFwdWsBase + need || stream_capturing(st)) return false;
  return coop_fits((const void*)pre_fwd_coop_kernel<32, false>, CoCfg<32>::THREADS, 0);
}

// The fused post + pre forward in one pass (pre_fwd_coop_kernel with POST):
// where the single-pass pre forward applies to x_next's shape, and x,
// h_out, x_next and y are 16-byte aligned, x_next is formed in the kernel
// and written once; *used says whether it ran.
int post_pre_fwd_single_pass(const void* x, const float* h_res, const void* h_out, const float* h_post,
                             const void* phi, const float* alpha, const float* base, float norm_eps, float hc_eps,
                             float clamp_min, float clamp_max, int32_t iter_times, void* x_next, void* y,
                             float* post_out, float* comb_frag, float* inv_rms, float* mixes, float* h_res_logits,
                             float* pre, void* workspace, size_t workspace_bytes, int32_t* status, int64_t T,
                             int32_t D, hipStream_t st, bool* used) {
  *used = false;
  constexpr int N = 4;
  if (!pre_fwd_single_pass_applies(x, MHC_DTYPE_BF16, phi, MHC_DTYPE_BF16, y, workspace_bytes, T, N, D, st) ||
      !aligned16(h_out) || !aligned16(x_next))
    return MHC_OK;
  const int M = 2 * N + N * N;
  const int64_t K = (int64_t)N * D;
  PreFwdArgs a{};
  a.x = x;
  int rc = prepare_phi_planes(phi, MHC_DTYPE_BF16, M, K, workspace, workspace_bytes, &a.phi, &a.phi_ld,
                              &a.phi_plane_stride, &a.phi_planes, st);
  if (rc) return rc;
  a.alpha = alpha;
  a.base = base;
  a.norm_eps = norm_eps;
  a.hc_eps = hc_eps;
  a.cmin = clamp_min;
  a.cmax = clamp_max;
  a.apply_clamp = (clamp_min != 0.0f || clamp_max != 0.0f) ? 1 : 0;
  a.iters = iter_times;
  a.y = y;
  a.post_out = post_out;
  a.comb = comb_frag;
  a.inv_rms = inv_rms;
  a.mixes = mixes;
  a.logits = h_res_logits;
  a.pre = pre;
  a.T = T;
  a.D = D;
  a.status_out = status;
  a.x_next_nan = x_next;
  CoopArgs post{};
  post.h_out = static_cast<const bf16_t*>(h_out);
  post.h_res = h_res;
  post.h_post = h_post;
  post.x_next = static_cast<bf16_t*>(x_next);
  return launch_pre_fwd_coop_x<false, true>(a, workspace, workspace_bytes, st, used, &post);
}
}  // namespace mhc

extern "C" int mhc_pre_fwd_ex(const void* x, int32_t x_dtype, const void* phi, int32_t phi_dtype,
                              const float* alpha, const float* base, float norm_eps, float hc_eps,
                              float clamp_min, float clamp_max, int32_t iter_times, void* y,
                              float* post_out, float* comb_frag, float* inv_rms, float* mixes,
                              float* h_res_logits, float* pre, float* x_scaled, void* workspace,
                              size_t workspace_bytes, int32_t* status, int64_t T, int32_t N, int32_t D,
                              void* stream) {
  clear_error();
  if (T < 0 || D <= 0 || N <= 0)
    return set_error(MHC_ERR_INVALID, "mhc_pre_fwd: bad shape T=%lld N=%d D=%d", (long long)T, N, D);
  if (int rc = check_tokens(T, "mhc_pre_fwd")) return rc;
  if (N != 4 && N != 8) return set_error(MHC_ERR_UNSUPPORTED, "mhc_pre_fwd: N=%d not supported (4, 8)", N);
  if (T == 0) return MHC_OK;
  if (!x || !phi || !alpha || !base || !y || !post_out || !comb_frag)
    return set_error(MHC_ERR_INVALID, "mhc_pre_fwd: null pointer");
  hipStream_t st = (hipStream_t)stream;
  const int M = 2 * N + N * N;
  const int64_t K = (int64_t)N * D;

  PreFwdArgs a{};
  a.x = x;
  int rc = prepare_phi_planes(phi, phi_dtype, M, K, workspace, workspace_bytes, &a.phi, &a.phi_ld,
                              &a.phi_plane_stride, &a.phi_planes, st);
  if (rc) return rc;
  a.alpha = alpha;
  a.base = base;
  a.norm_eps = norm_eps;
  a.hc_eps = hc_eps;
  a.cmin = clamp_min;
  a.cmax = clamp_max;
  a.apply_clamp = (clamp_min != 0.0f || clamp_max != 0.0f) ? 1 : 0;
  a.iters = iter_times;
  a.y = y;
  a.post_out = post_out;
  a.comb = comb_frag;
  a.inv_rms = inv_rms;
  a.mixes = mixes;
  a.logits = h_res_logits;
  a.pre = pre;
  a.x_scaled = x_scaled;
  a.T = T;
  a.D = D;
  a.status_out = status;
  const bool vec = (D % 8 == 0) && aligned16(x) && aligned16(y) && (!x_scaled || aligned16(x_scaled));
  const size_t y_ws = fwd_y_ws_bytes(T, N), ha_ws = heads_apart_bytes(T, N);
  const size_t dma_ws = kPreFwdWsBase + (ha_ws > y_ws ? ha_ws : y_ws);
  if (fwd_dma_usable(a, N, x_dtype == MHC_DTYPE_BF16, vec) && workspace && workspace_bytes >= dma_ws)
    return N == 4 ? launch_pre_fwd_dma<4>(a, workspace, workspace_bytes, st)
                  : launch_pre_fwd_dma<8>(a, workspace, workspace_bytes, st);
  switch (x_dtype) {
    case MHC_DTYPE_BF16: return dispatch_pre_fwd<bf16_t>(N, a, vec, st);
    case MHC_DTYPE_F16: return dispatch_pre_fwd<f16_t>(N, a, vec, st);
    case MHC_DTYPE_F32: return dispatch_pre_fwd<float>(N, a, vec, st);
  }
  return set_error(MHC_ERR_UNSUPPORTED, "mhc_pre_fwd: x dtype %d not supported", x_dtype);
}

extern "C" int mhc_pre_fwd(const void* x, int32_t x_dtype, const void* phi, int32_t phi_dtype,
                           const float* alpha, const float* base, float norm_eps, float hc_eps,
                           float clamp_min, float clamp_max, int32_t iter_times, void* y,
                           float* post_out, float* comb_frag, float* inv_rms, float* mixes,
                           float* h_res_logits, float* pre, float* x_scaled, void* workspace,
                           size_t workspace_bytes, int64_t T, int32_t N, int32_t D,
                           void* stream) {
  return mhc_pre_fwd_ex(x, x_dtype, phi, phi_dtype, alpha, base, norm_eps, hc_eps, clamp_min, clamp_max,
                        iter_times, y, post_out, comb_frag, inv_rms, mixes, h_res_logits, pre, x_scaled,
                        workspace, workspace_bytes, nullptr, T, N, D, stream);
}

extern "C" void mhc_debug_set_wait_limit(int64_t ticks) {
  coop_wait_limit_slot().store(ticks < 0 ? -1 : ticks, std::memory_order_relaxed);
}

// ---- allocation-free variant ------------------------------------------------
// mhc_pre_fwd_noalloc runs mhc_pre_fwd with its workspace in `scratch`, a
// static device array of MHC_PRE_FWD_SCRATCH_BYTES: every GPU the library runs
// on holds its own copy (the code object's zero-initialised data) until the
// process ends.  In host code the name `scratch` is a host-side stand-in, not
// a device address; the device address of the current GPU's copy comes from
// hipGetSymbolAddress, once per device, and only that address is passed on.
// Nothing in the workspace has to start at zero: every kernel writes the
// parts it later reads within the same call.  Calls that overlap on one GPU
// (two streams, two threads) share the array and race.
namespace mhc {

static __device__ __align__(256) unsigned char scratch[MHC_PRE_FWD_SCRATCH_BYTES];

// Device address of `scratch` on device `dev` (the current device), looked up
// on the first call for that device and cached.
static void* pre_fwd_scratch(int dev, int* rc) {
  static std::atomic<void*> cache[64];
  if (dev < 0 || dev >= 64) {
    *rc = set_error(MHC_ERR_UNSUPPORTED, "mhc_pre_fwd_noalloc: device %d above the 64 supported", dev);
    return nullptr;
  }
  void* p = cache[dev].load(std::memory_order_acquire);
  if (p) return p;
  const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess || !p) {
    *rc = set_error(MHC_ERR_HIP, "mhc_pre_fwd_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                    hipGetErrorString(e));
    return nullptr;
  }
  cache[dev].store(p, std::memory_order_release);
  return p;
}

}  // namespace mhc

extern "C" int mhc_pre_fwd_noalloc(const void* x, int32_t x_dtype, const void* phi, int32_t phi_dtype,
                                   const float* alpha, const float* base, float norm_eps, float hc_eps,
                                   float clamp_min, float clamp_max, int32_t iter_times, void* y,
                                   float* post_out, float* comb_frag, float* inv_rms, float* mixes,
                                   float* h_res_logits, float* pre, float* x_scaled, int64_t T, int32_t N,
                                   int32_t D, void* stream) {
  clear_error();
  if (T < 0 || D <= 0 || N <= 0)
    return set_error(MHC_ERR_INVALID, "mhc_pre_fwd_noalloc: bad shape T=%lld N=%d D=%d", (long long)T, N, D);
  // the two-pass forms fit in less; the single-pass one runs when it fits too
  const size_t need = pre_fwd_ws_min(T, N, D, phi_dtype);
  if (need > (size_t)MHC_PRE_FWD_SCRATCH_BYTES)
    return set_error(MHC_ERR_INVALID,
                     "mhc_pre_fwd_noalloc: T=%lld N=%d D=%d needs %zu bytes of workspace, above the %zu of "
                     "its static scratch (use mhc_pre_fwd with a workspace)",
                     (long long)T, N, D, need, (size_t)MHC_PRE_FWD_SCRATCH_BYTES);
  void* ws = nullptr;
  if (T > 0) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess)
      return set_error(MHC_ERR_HIP, "mhc_pre_fwd_noalloc: no current device");
    if (stream) {  // the scratch looked up below belongs to the current device
      int sdev = -1;
      if (hipStreamGetDevice((hipStream_t)stream, &sdev) != hipSuccess || sdev != dev)
        return set_error(MHC_ERR_INVALID, "mhc_pre_fwd_noalloc: stream of device %d, current device %d", sdev,
                         dev);
    }
    int rc = MHC_OK;
    ws = pre_fwd_scratch(dev, &rc);
    if (!ws) return rc;
  }
  return mhc_pre_fwd(x, x_dtype, phi, phi_dtype, alpha, base, norm_eps, hc_eps, clamp_min, clamp_max, iter_times,
                     y, post_out, comb_frag, inv_rms, mixes, h_res_logits, pre, x_scaled, ws,
                     (size_t)MHC_PRE_FWD_SCRATCH_BYTES, T, N, D, stream);
}
