// mhc_pre_clamp_sinkhorn backward.
//
// Semantics: torch autograd of mhc_pre_clamp_sinkhorn_ref, as the reference's
// mhc_pre_clamp_sinkhorn_backward_ref does
// (src/mhc_pre_clamp_sinkhorn_backward.py:1397-1453), for the loss
// <grad_y, y> + <grad_post_out, post_out> + <grad_comb_frag, comb_frag>.
//
// Kernel A (pre_bwd_small_kernel), a block per 16 tokens:
//   grad_pre[t,n] = <grad_y[t,:], x[t,n,:]>                (bf16 rows at
//   T >= 16384: the sums of pre_bwd_gpre_dma_kernel, a wave per token over
//   an LDS ring; smaller T: summed in fixed order from the partials of
//   pre_bwd_gpre_kernel, a block per (token, 2048 columns); N = 4 in other
//   dtypes at T >= 16384: a wave per token here)
//   Sinkhorn / softmax / clamp / sigmoid-head VJP, lane per matrix element
//   -> grad_mixes (T,M) and scale[t] = -inv^2 * <grad_mixes, mixes> / (N*D)
//   (because <x, grad_mixes @ phi> = <grad_mixes, mixes> / inv), plus a
//   per-block partial of grad_alpha / grad_base (fixed summation order).
// Kernel B (pre_bwd_main_kernel), a block per (256 k-columns, token split):
//   gs = grad_mixes @ phi on MFMA (A = phi^T rows kept in registers,
//   B = grad_mixes rows from LDS), then
//   grad_x = grad_y * pre[n] + inv * gs + scale * x, written once;
//   grad_phi partial += (grad_mixes * inv)^T @ x on MFMA over 32-token
//   sub-tiles staged in LDS.
// Kernels C: deterministic reductions of the grad_phi split partials and of
// the grad_alpha / grad_base block partials (no atomics anywhere).
#include <type_traits>

#include "mhc_launch.hpp"
#include "pre_common.hpp"
#include "pre_host.hpp"
#include "sinkhorn.hpp"

namespace mhc {

constexpr int kBwdTile = 16;
constexpr int kBwdThreads = 256;
constexpr int kMainKC = 256;  // k columns per main-kernel block (all N streams x KC/N widths)
constexpr int kMainTS = 32;   // tokens per main-kernel sub-tile
constexpr int kMaxSplits = 16;

// ---------------------------------------------------------------------------
// Kernel A
// ---------------------------------------------------------------------------
struct PreBwdSmallArgs {
  const void* x;
  const void* gy;
  const float* mixes;
  const float* inv_rms;
  const float* alpha;
  const float* base;
  const float* gpost;
  const float* gcomb;
  float hc_eps, cmin, cmax;
  int apply_clamp;
  int iters;
  const float* pre;
  float* gm;       // (T, M) fp32, or null
  float* scale;    // (T,), or null
  uint16_t* gmP;   // [2][T][MP32] bf16 planes of grad_mixes, or null
  int64_t gmP_plane;
  uint16_t* gTw;   // [ceil(T/16)][MT][64][2][4] bf16 planes of grad_mixes * inv
  float4* coef;    // (T, N) {pre, inv, scale, 0}, or null
  float* partial;  // (gridDim.x, 3 + M)
  float* sink_scratch;
  int64_t sink_stride;
  const float* gpre_part;  // [T][gpre_chunks][N] grad_pre partials, or null
  int gpre_chunks;
  float* gpre_buf;         // the workspace's partials region (host side: the LDS-pipelined grad_pre)
  float* coefX;            // single-pass form (N = 4): (T, 16) per-token records, see below
  int comp;                // compensated (Neumaier) sums of the block partials
  int64_t T;
  int D;
};

// Neumaier's compensated step: s + c tracks the exact sum of the added values
// (the error of each rounded addition is collected in c).
__device__ __forceinline__ void neumaier_add(float& s, float& c, float v) {
  const float t = s + v;
  c += fabsf(s) >= fabsf(v) ? (s - t) + v : (v - t) + s;
  s = t;
}

// Kahan's step (4 operations; c is the negated running error, so the sum is
// s - c): used per 32-token tile in the grad_phi kernel, where the VALU is the
// bound and each added tile is the sum of many products.
__device__ __forceinline__ void kahan_add(float& s, float& c, float v) {
  const float y = v - c;
  const float t = s + y;
  c = (t - s) - y;
  s = t;
}

// grad_pre partials for small T, where a block per 16 tokens leaves most of
// the chip idle and each wave streams (N + 1) * D elements serially: a block
// per (token, 2048-column chunk) writes part[t][chunk][n] =
// sum over its columns of grad_y[t,d] * x[t,n,d] (per-thread FMA chain over
// 8 columns, wave_sum, then the 4 waves in order).
constexpr int kGpreCols = kBwdThreads * 8;

// Blocks in x: at most kGpreGridT, each looping over the tokens
// blockIdx.x, blockIdx.x + gridDim.x, ..., so the launch stays far below the
// 2^32 work-items of a dispatch at any T.
constexpr int64_t kGpreGridT = 65536;

template <int N, typename S, bool VEC>
__global__ __launch_bounds__(kBwdThreads) void pre_bwd_gpre_kernel(const void* xv, const void* gyv, float* part,
                                                                   int64_t T, int D) {
  __shared__ float red[kBwdThreads / kWave][N];
  const S* __restrict__ x = static_cast<const S*>(xv);
  const S* __restrict__ gy = static_cast<const S*>(gyv);
  const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid >> 6;
  const int64_t d = (int64_t)blockIdx.y * kGpreCols + tid * 8;
  const bool ok = d < D;
  for (int64_t tok = blockIdx.x; tok < T; tok += gridDim.x) {  // uniform over the block
    float acc[N];
    float g8[8];
    load8f<S, VEC>(gy + tok * D, d, D, ok, g8);
#pragma unroll
    for (int n = 0; n < N; ++n) {
      float x8[8];
      load8f<S, VEC>(x + (tok * N + n) * D, d, D, ok, x8);
      acc[n] = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[n] = fmaf(g8[i], x8[i], acc[n]);
    }
#pragma unroll
    for (int n = 0; n < N; ++n) acc[n] = wave_sum(acc[n]);
    if (lane == 0) {
#pragma unroll
      for (int n = 0; n < N; ++n) red[wave][n] = acc[n];
    }
    __syncthreads();
    if (tid < N) {
      float s = red[0][tid];
#pragma unroll
      for (int w = 1; w < kBwdThreads / kWave; ++w) s += red[w][tid];
      part[(tok * gridDim.y + blockIdx.y) * N + tid] = s;
    }
    __syncthreads();  // red is rewritten for the next token
  }
}

// grad_pre for large T, LDS-pipelined (bf16, 16-byte rows): every wave of a
// persistent grid streams its tokens w, w + W, ... through a private ring of
// S slots, one slot = the token's N x rows and its grad_y row over 512
// columns (one 1 KB direct-to-LDS load per row, lane l -> columns 8l..8l+7),
// loaded S - 1 slots ahead; a wave reads back only what its own loads wrote,
// so there are no barriers.  Each lane accumulates its columns' products in
// kernel A's order (per 512-column chunk, fmaf over its 8 columns) and the
// token's N sums leave through wave_sum, as in kernel A's own loop, to
// part[t][n] (one chunk), which kernel A then reads: the same bits as its
// wave-per-token loop, the reads at the direct-to-LDS rate.
constexpr int kGpreDmaWaves = 4;
template <int N> struct GpreDmaCfg {
  static constexpr int R = N + 1;          // slot rows: x[0..N-1], grad_y
  static constexpr int S = N == 4 ? 6 : 4;  // 4 waves x S x R KB: 120 / 144 KB
};

template <int N>
__global__ __launch_bounds__(kWave * kGpreDmaWaves) void pre_bwd_gpre_dma_kernel(const bf16_t* __restrict__ x,
                                                                                 const bf16_t* __restrict__ gy,
                                                                                 float* __restrict__ part, int64_t T,
                                                                                 int D) {
  constexpr int R = GpreDmaCfg<N>::R, S = GpreDmaCfg<N>::S;
  // slot j's loads have landed once at most VM newer vector memory operations
  // are outstanding (the loads of the S - 2 slots issued after it; a token's
  // sums stored in between only add newer ones)
  constexpr int VM = (S - 2) * R;
  static_assert(VM < 64 && R % 4 == 1, "vmcnt range; slot rows 4k + 1");
  __shared__ u32x4 ring[kGpreDmaWaves * S * R * kWave];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t gw = (int64_t)blockIdx.x * kGpreDmaWaves + wave, W = (int64_t)gridDim.x * kGpreDmaWaves;
  const int ncb = (D + 511) / 512;
  const int64_t ntok = (T - gw + W - 1) / W;
  if (ntok <= 0) return;  // this wave only: no barriers below
  const int64_t J = ntok * ncb;
  const uint32_t wring = lds_addr(ring) + (uint32_t)(wave * S * R * 1024);
  const int64_t ND = (int64_t)N * D;

  int64_t itok = gw;
  int icb = 0;
  auto issue = [&](int64_t j) {
    const uint32_t slot = wring + (uint32_t)((j % S) * R * 1024);
    const int col = icb * 512 + 8 * lane;
    const auto rx = rows_rsrc(x + itok * ND, ND * 2);
    const auto rg = rows_rsrc(gy + itok * D, (int64_t)D * 2);
#pragma unroll
    for (int n = 0; n < N; ++n)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_void_t*)(uintptr_t)(slot + n * 1024), 16,
                                               col < D ? (uint32_t)(((int64_t)n * D + col) * 2) : kBufferOob,
                                               0, 0, 2 /* nt */);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rg, (lds_void_t*)(uintptr_t)(slot + N * 1024), 16,
                                             col < D ? (uint32_t)(col * 2) : kBufferOob, 0, 0, 2);
    if (++icb == ncb) {
      icb = 0;
      itok += W;
    }
  };
  for (int64_t j = 0; j < S - 1 && j < J; ++j) issue(j);

  int64_t ctok = gw;
  int ccb = 0;
  float acc[N];
#pragma unroll
  for (int n = 0; n < N; ++n) acc[n] = 0.f;
  for (int64_t j = 0; j < J; ++j) {
    if (j + S - 2 < J)
      wait_vmcnt<VM>();
    else
      wait_vmcnt<0>();
    asm volatile("" ::: "memory");
    // the next loads reuse the slot this wave read (and waited for) last iteration
    if (j + S - 1 < J) issue(j + S - 1);
    u32x4 v[R];
    read_slot<R>(v, wring + (uint32_t)((j % S) * R * 1024) + lane * 16);
    float g8[8];
    Store<bf16_t>::unpack(v[N], g8);
#pragma unroll
    for (int n = 0; n < N; ++n) {
      float x8[8];
      Store<bf16_t>::unpack(v[n], x8);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[n] = fmaf(g8[i], x8[i], acc[n]);
    }
    if (++ccb == ncb) {
#pragma unroll
      for (int n = 0; n < N; ++n) acc[n] = wave_sum(acc[n]);
      if (lane == 0) {
#pragma unroll
        for (int n = 0; n < N; ++n) part[ctok * N + n] = acc[n];
      }
#pragma unroll
      for (int n = 0; n < N; ++n) acc[n] = 0.f;
      ccb = 0;
      ctok += W;
    }
  }
}

// SP (the single-pass backward, pre_bwd_coop.hpp): grad_pre is not known
// yet, so the pre head's part of grad_mixes is left to the single-pass
// kernel: grad_mixes[t, n < N] and its terms of scale, grad_alpha[0] and
// grad_base[n < N] are zero here, and coefX[t] = {pre[0..3],
// sp(1 - sp)[0..3] (sp = sigmoid(mixes[n] * alpha[0] + base[n])),
// mixes[0..3], inv_rms, scale without the pre head, 0, 0} carries what the
// single-pass kernel needs to add them (grad_mixes[t, n] = grad_pre[t, n] *
// alpha[0] * sp(1 - sp)).
template <int N, typename S, bool VEC, bool SP = false>
__global__ __launch_bounds__(kBwdThreads) void pre_bwd_small_kernel(PreBwdSmallArgs a) {
  static_assert(!SP || N == 4, "single-pass records hold four streams");
  using PD = PreDims<N>;
  constexpr int M = PD::M, L = N * N, C = 3 + M;
  __shared__ float gp_sh[kBwdTile][N];
  __shared__ float contrib[kBwdTile][C + 1];

  const S* __restrict__ x = static_cast<const S*>(a.x);
  const S* __restrict__ gy = static_cast<const S*>(a.gy);
  const int D = a.D;
  const int64_t K = (int64_t)N * D;
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t t0 = (int64_t)blockIdx.x * kBwdTile;

  // ---- grad_pre: summed from the split kernel's partials, or a wave per token
  if constexpr (SP) {
    if (tid < kBwdTile * N) gp_sh[tid / N][tid % N] = 0.f;
  } else if (a.gpre_part) {
    if (tid < kBwdTile * N) {
      const int tt = tid / N, n = tid % N;
      const int64_t tok = t0 + tt;
      float s = 0.f;
      if (tok < a.T) {
        const float* pp = a.gpre_part + tok * a.gpre_chunks * N + n;
#pragma unroll 4
        for (int c = 0; c < a.gpre_chunks; ++c) s += pp[c * N];
      }
      gp_sh[tt][n] = s;
    }
  } else {
    for (int q = 0; q < kBwdTile / 4; ++q) {
      const int tt = wave + 4 * q;
      const int64_t tok = t0 + tt;
      float acc[N];
#pragma unroll
      for (int n = 0; n < N; ++n) acc[n] = 0.f;
      if (tok < a.T) {
        for (int64_t d = (int64_t)lane * 8; d < D; d += kWave * 8) {
          float g8[8];
          load8f<S, VEC>(gy + tok * D, d, D, true, g8);
#pragma unroll
          for (int n = 0; n < N; ++n) {
            float x8[8];
            load8f<S, VEC>(x + (tok * N + n) * D, d, D, true, x8);
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[n] = fmaf(g8[i], x8[i], acc[n]);
          }
        }
      }
#pragma unroll
      for (int n = 0; n < N; ++n) acc[n] = wave_sum(acc[n]);
      if (lane == 0) {
#pragma unroll
        for (int n = 0; n < N; ++n) gp_sh[tt][n] = acc[n];
      }
    }
  }
  __syncthreads();

  // ---- small stage, lane per N x N element --------------------------------
  constexpr int TPP = kBwdThreads / L, PASSES = kBwdTile / TPP;
  const float a0 = a.alpha[0], a1 = a.alpha[1], a2 = a.alpha[2];
#pragma unroll
  for (int ps = 0; ps < PASSES; ++ps) {
    const int tt = ps * TPP + tid / L;
    const int e = tid % L;
    const int64_t tok = t0 + tt;
    const bool ok = tok < a.T;
    const float* mrow = a.mixes + (ok ? tok * M : 0);
    const float ml = ok ? mrow[2 * N + e] : 0.f;
    const float logit = ml * a2 + a.base[2 * N + e];
    const float lc = clamp_logit(logit, a.apply_clamp, a.cmin, a.cmax);
    const float g = ok ? a.gcomb[tok * L + e] : 0.f;
    float dlc;
    if (a.iters <= kSinkRegIters)
      dlc = sinkhorn_vjp_regs<N>(lc, g, a.hc_eps, a.iters);
    else
      dlc = sinkhorn_vjp_scratch<N>(lc, g, a.hc_eps, a.iters,
                                    a.sink_scratch + ((int64_t)blockIdx.x * kBwdTile + tt) * L + e,
                                    a.sink_stride);
    // torch.clamp passes the gradient where lo <= logit <= hi (inclusive)
    if (a.apply_clamp && !(logit >= a.cmin && logit <= a.cmax)) dlc = 0.f;
    const float gml = dlc * a2;

    float gmh = 0.f, mh = 0.f, dz = 0.f;
    if (e < 2 * N) {
      mh = ok ? mrow[e] : 0.f;
      if (e < N) {
        const float sp = sigmoidf_(mh * a0 + a.base[e]);
        dz = gp_sh[tt][e] * sp * (1.0f - sp);
        gmh = dz * a0;
        if constexpr (SP) {
          if (ok) {
            a.coefX[tok * 16 + e] = a.pre[tok * N + e];
            a.coefX[tok * 16 + 4 + e] = sp * (1.0f - sp);
            a.coefX[tok * 16 + 8 + e] = mh;
          }
        }
      } else {
        const float so = sigmoidf_(mh * a1 + a.base[e]);
        const float gpo = ok ? a.gpost[tok * N + (e - N)] : 0.f;
        dz = gpo * 2.0f * so * (1.0f - so);
        gmh = dz * a1;
      }
    }
    const float inv = ok ? a.inv_rms[tok] : 0.f;
    if (ok && a.gm) {
      a.gm[tok * M + 2 * N + e] = gml;
      if (e < 2 * N) a.gm[tok * M + e] = gmh;
    }
    if (a.gmP) {
      // operand layouts of the streaming kernels: grad_mixes as bf16 planes
      // [2][T][MP32], and g = grad_mixes * inv as token-transposed 16-token
      // tiles [T/16][MT][64][2][4]: element m of token 16*tile + 4*qq + j
      // sits at [tile][m / 16][m % 16 + 16*qq][plane][j], so MFMA lane
      // (m % 16, qq) finds both planes of its 4 tokens in 16 contiguous
      // bytes.  Padding rows m >= M are zero, and so are the g columns of
      // the padding tokens T..16*ceil(T/16)-1 (this grid covers exactly
      // those tokens).
      constexpr int MP32 = PD::MP32, MP = PD::MP;
      uint16_t* gTw = a.gTw + (tok >> 4) * (PD::MT * 64 * 8) + ((tok & 15) >> 2) * 16 * 8 + (tok & 3);
      auto gtw = [&](int m, int g) -> uint16_t& { return gTw[((m >> 4) * 64 + (m & 15)) * 8 + g * 4]; };
      uint32_t hi, lo;
      if (ok) {
        uint16_t* gmP = a.gmP + tok * MP32;
        split2_bf16(gml, hi, lo);
        gmP[2 * N + e] = (uint16_t)hi;
        gmP[a.gmP_plane + 2 * N + e] = (uint16_t)lo;
        if (e < 2 * N) {
          split2_bf16(gmh, hi, lo);
          gmP[e] = (uint16_t)hi;
          gmP[a.gmP_plane + e] = (uint16_t)lo;
        }
        if (e < MP32 - M) {
          gmP[M + e] = 0;
          gmP[a.gmP_plane + M + e] = 0;
        }
      }
      split2_bf16(ok ? gml * inv : 0.f, hi, lo);
      gtw(2 * N + e, 0) = (uint16_t)hi;
      gtw(2 * N + e, 1) = (uint16_t)lo;
      if (e < 2 * N) {
        split2_bf16(ok ? gmh * inv : 0.f, hi, lo);
        gtw(e, 0) = (uint16_t)hi;
        gtw(e, 1) = (uint16_t)lo;
      }
      if (e < MP - M) {
        gtw(M + e, 0) = 0;
        gtw(M + e, 1) = 0;
      }
    }
    const float sdot = group_sum<L - 1>(gml * ml + gmh * mh);
    const float c0 = group_sum<L - 1>(e < N ? dz * mh : 0.f);
    const float c1 = group_sum<L - 1>((e >= N && e < 2 * N) ? dz * mh : 0.f);
    const float c2 = group_sum<L - 1>(dlc * ml);
    const float scale = -inv * inv * sdot / (float)K;
    if (ok && a.coef && e < N) a.coef[tok * N + e] = float4{a.pre[tok * N + e], inv, scale, 0.f};
    if constexpr (SP) {
      if (ok && e == 0) *reinterpret_cast<float4*>(a.coefX + tok * 16 + 12) = float4{inv, scale, 0.f, 0.f};
    }
    if (e == 0) {
      if (ok && a.scale) a.scale[tok] = scale;
      contrib[tt][0] = c0;
      contrib[tt][1] = c1;
      contrib[tt][2] = c2;
    }
    contrib[tt][3 + 2 * N + e] = dlc;
    if (e < 2 * N) contrib[tt][3 + e] = dz;
  }
  __syncthreads();

  for (int c = tid; c < C; c += kBwdThreads) {
    float s = 0.f;
    if (a.comp) {
      float cc = 0.f;
#pragma unroll
      for (int tt = 0; tt < kBwdTile; ++tt) neumaier_add(s, cc, contrib[tt][c]);
      s += cc;
    } else {
#pragma unroll
      for (int tt = 0; tt < kBwdTile; ++tt) s += contrib[tt][c];
    }
    a.partial[(int64_t)blockIdx.x * C + c] = s;
  }
}

// ---------------------------------------------------------------------------
// Kernel B
// ---------------------------------------------------------------------------
struct PreBwdMainArgs {
  const void* x;
  const void* gy;
  const uint16_t* phiT;  // [P][K][MP32]
  int64_t phiT_plane_stride;
  int phi_planes;
  const float* gm;
  const float* inv_rms;
  const float* pre;
  const float* scale;
  void* gx;
  float* gphi_part;  // [nsplit][M][K]
  int64_t T;
  int D;
  int64_t tok_per_split;
};

template <typename S> struct Raw { typedef uint16_t type; };
template <> struct Raw<float> { typedef float type; };

template <typename S> __device__ __forceinline__ float raw_to_f32(typename Raw<S>::type v) {
  return Store<S>::to_f32(v);
}
template <> __device__ __forceinline__ float raw_to_f32<float>(float v) { return v; }

// 8 raw elements of a row (element-wise with bound `lim` unless VEC)
template <typename S, bool VEC>
__device__ __forceinline__ void copy8_to_lds(const S* src, int64_t lim, bool ok,
                                             typename Raw<S>::type* dst) {
  typedef typename Raw<S>::type R;
  if constexpr (VEC) {
    if constexpr (sizeof(S) == 2) {
      const u32x4 v = (ok && lim >= 8) ? ld16nt(src) : zero4();
      st16(dst, v);
    } else {
      u32x4 v0 = zero4(), v1 = zero4();
      if (ok && lim >= 8) {
        v0 = ld16nt(src);
        v1 = ld16nt(src + 4);
      }
      st16(dst, v0);
      st16(dst + 4, v1);
    }
  } else {
    const R* s = reinterpret_cast<const R*>(src);
#pragma unroll
    for (int i = 0; i < 8; ++i) dst[i] = (ok && i < lim) ? s[i] : (R)0;
  }
}

template <int N, typename S, bool VEC>
__global__ __launch_bounds__(256) void pre_bwd_main_kernel(PreBwdMainArgs a) {
  using PD = PreDims<N>;
  typedef typename Raw<S>::type R;
  constexpr int M = PD::M, MT = PD::MT, MP = PD::MP, MK = PD::MK, MP32 = PD::MP32;
  constexpr int KC = kMainKC, DC = KC / N, TS = kMainTS;
  constexpr int XP = XGroup<S>::PLANES;
  constexpr int XPITCH = KC + 8, GPITCH = DC + 8, MPITCH = MP32 + 8, TPITCH = TS + 8;

  __shared__ __attribute__((aligned(16))) R xs[TS][XPITCH];
  __shared__ __attribute__((aligned(16))) R gys[TS][GPITCH];
  __shared__ __attribute__((aligned(16))) uint16_t gmS[2][TS][MPITCH];
  __shared__ __attribute__((aligned(16))) uint16_t gT[2][MP][TPITCH];
  __shared__ float pre_sh[TS][N];
  __shared__ float inv_sh[TS], scale_sh[TS];

  const S* __restrict__ x = static_cast<const S*>(a.x);
  const S* __restrict__ gy = static_cast<const S*>(a.gy);
  S* __restrict__ gx = static_cast<S*>(a.gx);
  const int D = a.D;
  const int64_t K = (int64_t)N * D;
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, kq = lane >> 4;
  const int d0 = blockIdx.x * DC;
  const int64_t tbeg = (int64_t)blockIdx.y * a.tok_per_split;
  const int64_t tend = (tbeg + a.tok_per_split < a.T) ? tbeg + a.tok_per_split : a.T;
  const int P = a.phi_planes;

  // padding rows/columns of the operand tiles stay zero
  for (int i = tid; i < 2 * TS * MPITCH; i += 256) (&gmS[0][0][0])[i] = 0;
  for (int i = tid; i < 2 * MP * TPITCH; i += 256) (&gT[0][0][0])[i] = 0;

  // A operands of gs^T = phi^T-rows x grad_mixes^T: MFMA row rr of k-tile q maps to
  // wave column 16*(rr/4) + 4*q + rr%4, so each lane's outputs cover 16
  // consecutive columns.
  u32x4 aphi[4][MK][2];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int col = wave * 64 + 16 * (r >> 2) + 4 * q + (r & 3);
    const int n = col / DC, dd = col - (col / DC) * DC;
    const bool ok = d0 + dd < D;
    const int64_t kg = (int64_t)n * D + d0 + dd;
#pragma unroll
    for (int mk = 0; mk < MK; ++mk)
#pragma unroll
      for (int p = 0; p < 2; ++p)
        aphi[q][mk][p] = (ok && p < P)
                             ? ld16(a.phiT + p * a.phiT_plane_stride + kg * MP32 + 32 * mk + 8 * kq)
                             : zero4();
  }

  floatx4 ph[4][MT];
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) ph[q][mt] = floatx4{0.f, 0.f, 0.f, 0.f};

  for (int64_t tb = tbeg; tb < tend; tb += TS) {
    __syncthreads();  // previous sub-tile fully consumed
    // ---- stage the sub-tile -------------------------------------------------
    constexpr int UPT = N * (DC / 8);  // 8-element units per token row chunk
    for (int u = tid; u < TS * UPT; u += 256) {
      const int tt = u / UPT, rem = u - (u / UPT) * UPT;
      const int n = rem / (DC / 8), dd = (rem - (rem / (DC / 8)) * (DC / 8)) * 8;
      const int64_t tok = tb + tt;
      copy8_to_lds<S, VEC>(x + (tok * N + n) * D + d0 + dd, (int64_t)D - d0 - dd, tok < tend,
                           &xs[tt][n * DC + dd]);
    }
    for (int u = tid; u < TS * (DC / 8); u += 256) {
      const int tt = u / (DC / 8), dd = (u - (u / (DC / 8)) * (DC / 8)) * 8;
      const int64_t tok = tb + tt;
      copy8_to_lds<S, VEC>(gy + tok * D + d0 + dd, (int64_t)D - d0 - dd, tok < tend, &gys[tt][dd]);
    }
    for (int u = tid; u < TS * M; u += 256) {
      const int tt = u / M, m = u - (u / M) * M;
      const int64_t tok = tb + tt;
      const bool ok = tok < tend;
      const float v = ok ? a.gm[tok * M + m] : 0.f;
      const float inv = ok ? a.inv_rms[tok] : 0.f;
      uint32_t hi, lo;
      split2_bf16(v, hi, lo);
      gmS[0][tt][m] = (uint16_t)hi;
      gmS[1][tt][m] = (uint16_t)lo;
      split2_bf16(v * inv, hi, lo);
      gT[0][m][tt] = (uint16_t)hi;
      gT[1][m][tt] = (uint16_t)lo;
    }
    for (int u = tid; u < TS * N; u += 256) {
      const int tt = u / N, n = u - (u / N) * N;
      const int64_t tok = tb + tt;
      pre_sh[tt][n] = tok < tend ? a.pre[tok * N + n] : 0.f;
    }
    if (tid < TS) {
      const int64_t tok = tb + tid;
      inv_sh[tid] = tok < tend ? a.inv_rms[tok] : 0.f;
      scale_sh[tid] = tok < tend ? a.scale[tok] : 0.f;
    }
    __syncthreads();

    // ---- gs and grad_x ---------------------------------------------------------
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int tt = 16 * h + r;
      floatx4 gs[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) gs[q] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int mk = 0; mk < MK; ++mk) {
        const u32x4 b0 = *reinterpret_cast<const u32x4*>(&gmS[0][tt][32 * mk + 8 * kq]);
        const u32x4 b1 = *reinterpret_cast<const u32x4*>(&gmS[1][tt][32 * mk + 8 * kq]);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          gs[q] = mfma16x16x32(as_bf16x8(aphi[q][mk][0]), as_bf16x8(b0), gs[q]);
          gs[q] = mfma16x16x32(as_bf16x8(aphi[q][mk][0]), as_bf16x8(b1), gs[q]);
          if (P > 1) gs[q] = mfma16x16x32(as_bf16x8(aphi[q][mk][1]), as_bf16x8(b0), gs[q]);
        }
      }
      const int col0 = wave * 64 + 16 * kq;
      const int n = col0 / DC, dd0 = col0 - (col0 / DC) * DC;
      const float pn = pre_sh[tt][n], iv = inv_sh[tt], sc = scale_sh[tt];
      float o[16];
#pragma unroll
      for (int c = 0; c < 16; ++c) {
        const float xv = raw_to_f32<S>(xs[tt][col0 + c]);
        const float gv = raw_to_f32<S>(gys[tt][dd0 + c]);
        o[c] = fmaf(sc, xv, fmaf(iv, gs[c >> 2][c & 3], gv * pn));
      }
      const int64_t tok = tb + tt;
      if (tok < tend) {
        S* dst = gx + (tok * N + n) * D + d0;
        store8<S, VEC>(dst, dd0, (int64_t)D - d0, o);
        store8<S, VEC>(dst, dd0 + 8, (int64_t)D - d0, o + 8);
      }
    }

    // ---- grad_phi partial += (grad_mixes*inv)^T @ x -------------------------
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int col = wave * 64 + 16 * q + r;
      float f[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) f[e] = raw_to_f32<S>(xs[8 * kq + e][col]);
      u32x4 bx[2];
      if constexpr (XP == 1) {
        // bf16: rebuild the operand from raw bits (exact)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          bx[0][i] = (uint32_t)xs[8 * kq + 2 * i][col] | ((uint32_t)xs[8 * kq + 2 * i + 1][col] << 16);
        bx[1] = zero4();
      } else {
        split8(f, bx[0], bx[1]);
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const u32x4 g0 = *reinterpret_cast<const u32x4*>(&gT[0][16 * mt + r][8 * kq]);
        const u32x4 g1 = *reinterpret_cast<const u32x4*>(&gT[1][16 * mt + r][8 * kq]);
        ph[q][mt] = mfma16x16x32(as_bf16x8(g0), as_bf16x8(bx[0]), ph[q][mt]);
        ph[q][mt] = mfma16x16x32(as_bf16x8(g1), as_bf16x8(bx[0]), ph[q][mt]);
        if constexpr (XP > 1) ph[q][mt] = mfma16x16x32(as_bf16x8(g0), as_bf16x8(bx[1]), ph[q][mt]);
      }
    }
  }

  // ---- write this split's grad_phi partial ---------------------------------
  float* part = a.gphi_part + (int64_t)blockIdx.y * M * K;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int col = wave * 64 + 16 * q + r;
    const int n = col / DC, dd = col - (col / DC) * DC;
    if (d0 + dd >= D) continue;
    const int64_t kg = (int64_t)n * D + d0 + dd;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int m = 16 * mt + 4 * kq + v;
        if (m < M) part[(int64_t)m * K + kg] = ph[q][mt][v];
      }
  }
}

// ---------------------------------------------------------------------------
// Kernel B, streaming form (bf16 activations, 16-byte aligned rows)
//
// A block has one wave per stream n and owns DW = 16*VC columns d of every
// stream; it walks 16-token tiles t = split, split + nsplit, ... so every
// block of the persistent grid gets the same work.  Lane (r = lane%16,
// q = lane/16) loads, for the 4 tokens 4q..4q+3 of a tile, the VC columns
// d0 + VC*r.. of x[t, n, :] and grad_y[t, :] (one coalesced load per row),
// i.e. a 4 x VC bf16 block held in registers:
//   * grad_phi (MFMA 16x16x16, reduction over the 16 tokens): the block is
//     transposed in registers (16-bit shuffles inside the lane) so that its
//     column c is a B operand (4 tokens of one column); A = (grad_mixes*inv)^T
//     read from token-transposed 16-token tiles.  MFMA instance c covers the
//     columns VC*r + c, r = 0..15.
//   * gs = grad_mixes @ phi (MFMA 16x16x32, reduction over m): A = the 16
//     tokens' grad_mixes rows, B = phi^T rows kept in registers for the whole
//     kernel.  Output lane (r, q) holds tokens 4q..4q+3 of columns VC*r + c:
//     exactly the rows of x and grad_y the lane loaded, so
//     grad_x = grad_y*pre + inv*gs + scale*x is formed and stored in place.
// No LDS and no barriers: each wave streams independently.  Used for N = 8;
// N = 4 takes the LDS-pipelined form below.
// ---------------------------------------------------------------------------
template <int N> struct StreamCfg {
  static constexpr int VC = (N == 4) ? 8 : 4;  // columns per lane
  static constexpr int DW = 16 * VC;           // columns per block and stream
};

constexpr int kStreamTile = 16;  // tokens per tile (MFMA K of the grad_phi product)
static_assert(kStreamTile == kBwdTile, "kernel A zero-fills the g tiles of the padding tokens");

struct PreBwdStreamArgs {
  const bf16_t* x;
  const bf16_t* gy;
  const uint16_t* phiT;  // [P][K][MP32]
  int64_t phiT_plane_stride;
  int phi_planes;
  const uint16_t* gmP;   // [2][T][MP32]
  int64_t gmP_plane;
  const uint16_t* gTw;   // [ceil(T/16)][MT][64][2][4]
  const float4* coef;    // (T, N) {pre, inv, scale, 0}
  bf16_t* gx;
  const bf16_t* gin;     // accumulating form (LDS-pipelined kernel): grad_x = gin + dL/dx
  float* gphi_part;      // [nsplit][M][K]
  int64_t T;
  int D;
  int nsplit;
};

template <int VD> struct RowVec;
template <> struct RowVec<4> { typedef u32x4 type; };
template <> struct RowVec<2> { typedef u32x2 type; };

typedef short short4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ floatx4 mfma16x16x16(const u32x2& a, const u32x2& b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(short4_t, a),
                                                  __builtin_bit_cast(short4_t, b), c, 0, 0, 0);
}

// Operands of one 16-token tile.
template <int N> struct StreamTile {
  static constexpr int VC = StreamCfg<N>::VC, VD = VC / 2;
  typedef typename RowVec<VD>::type Row;
  Row xr[4], gr[4];                   // x[t, n, cols] and grad_y[t, cols], tokens 4q..4q+3
  u32x4 gA[PreDims<N>::MK][2];        // grad_mixes row of token tb + r (A of gs), hi/lo
  u32x2 ga[PreDims<N>::MT][2];        // (grad_mixes*inv)^T, tokens 4q..4q+3 (A of grad_phi)
  float4 cf[4];                       // {pre[t,n], inv[t], scale[t]} of tokens 4q..4q+3
};

template <int N, int P>
__global__ __launch_bounds__(64 * N) void pre_bwd_stream_kernel(PreBwdStreamArgs a) {
  using PD = PreDims<N>;
  using Tile = StreamTile<N>;
  typedef typename Tile::Row Row;
  constexpr int M = PD::M, MT = PD::MT, MK = PD::MK, MP32 = PD::MP32;
  constexpr int VC = StreamCfg<N>::VC, DW = StreamCfg<N>::DW, VD = VC / 2;
  constexpr int TT = kStreamTile;

  const int lane = threadIdx.x & (kWave - 1);
  const int n = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, q = lane >> 4;
  const int D = a.D;
  const int64_t K = (int64_t)N * D, T = a.T;
  const int dl = blockIdx.x * DW + VC * r;  // first column d of this lane
  const bool colok = dl < D;                // D % VC == 0 on this path
  const int dlc = colok ? dl : 0;           // clamped column for branch-free loads
  const int64_t kcol = (int64_t)n * D + dl;

  u32x4 pb[VC][MK][P];
#pragma unroll
  for (int c = 0; c < VC; ++c)
#pragma unroll
    for (int mk = 0; mk < MK; ++mk)
#pragma unroll
      for (int p = 0; p < P; ++p)
        pb[c][mk][p] = colok ? ld16(a.phiT + p * a.phiT_plane_stride + (kcol + c) * MP32 + 32 * mk + 8 * q)
                             : zero4();

  floatx4 ph[MT][VC];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int c = 0; c < VC; ++c) ph[mt][c] = floatx4{0.f, 0.f, 0.f, 0.f};

  // Loads are unconditional from clamped addresses and their data is used
  // unmodified, so a tile's loads issue back to back and stay in flight
  // until compute_tile: a clamped x row meets zero columns of g (kernel A
  // zero-fills the padding tokens of the last tile), clamped gm rows and
  // coefficients only reach outputs of tokens >= T, which are not stored.
  // With one phi plane the x / grad_y rows (HBM) are loaded one tile ahead,
  // after the current tile's workspace operands (L2): vector loads complete
  // in issue order, so waiting for those operands leaves the next rows in
  // flight (N = 8, D = 2048: 1.49 -> 1.34 ms for the backward on MI355X).  A
  // whole second tile of operands would not fit the 256 VGPRs of two waves
  // per SIMD; with two phi planes even the rows spill (1.78 -> 2.14 ms), so
  // that form loads a tile and then computes it.
  auto load_rows = [&](int64_t tile, Row* xr, Row* gr) {
    const int64_t tg = tile * TT + 4 * q;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int64_t t = tg + e;
      const int64_t tc = t < T ? t : T - 1;
      xr[e] = __builtin_nontemporal_load(reinterpret_cast<const Row*>(a.x + (tc * N + n) * D + dlc));
      gr[e] = *reinterpret_cast<const Row*>(a.gy + tc * D + dlc);
    }
  };
  auto load_operands = [&](int64_t tile, Tile& tl) {
    const int64_t tb = tile * TT, tg = tb + 4 * q;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int64_t t = tg + e;
      const int64_t tc = t < T ? t : T - 1;
      tl.cf[e] = a.coef[tc * N + n];
    }
    const int64_t ts = tb + r;  // token of MFMA row r in the gs product
    const int64_t tsc = ts < T ? ts : T - 1;
#pragma unroll
    for (int mk = 0; mk < MK; ++mk)
#pragma unroll
      for (int g = 0; g < 2; ++g) tl.gA[mk][g] = ld16(a.gmP + g * a.gmP_plane + tsc * MP32 + 32 * mk + 8 * q);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const u32x4 v = ld16(a.gTw + ((tile * MT + mt) * 64 + lane) * 8);
      tl.ga[mt][0] = u32x2{v[0], v[1]};
      tl.ga[mt][1] = u32x2{v[2], v[3]};
    }
  };

  auto compute_tile = [&](int64_t tile, const Tile& tl) {
    const int64_t tg = tile * TT + 4 * q;
    // ---- grad_phi partial += g^T @ x over the tile's 16 tokens ----------
#pragma unroll
    for (int c = 0; c < VC; ++c) {
      // column c of the lane's 4 x VC block: tokens (2w, 2w+1) in dword w
      u32x2 xt;
#pragma unroll
      for (int w = 0; w < 2; ++w) {
        const uint32_t lo = tl.xr[2 * w][c >> 1], hi = tl.xr[2 * w + 1][c >> 1];
        xt[w] = (c & 1) ? ((lo >> 16) | (hi & 0xffff0000u)) : ((lo & 0xffffu) | (hi << 16));
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        ph[mt][c] = mfma16x16x16(tl.ga[mt][0], xt, ph[mt][c]);
        ph[mt][c] = mfma16x16x16(tl.ga[mt][1], xt, ph[mt][c]);
      }
    }
    // ---- gs = grad_mixes @ phi, then grad_x ---------------------------------
    floatx4 gs[VC];
#pragma unroll
    for (int c = 0; c < VC; ++c) {
      gs[c] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int mk = 0; mk < MK; ++mk) {
        gs[c] = mfma16x16x32(as_bf16x8(tl.gA[mk][0]), as_bf16x8(pb[c][mk][0]), gs[c]);
        gs[c] = mfma16x16x32(as_bf16x8(tl.gA[mk][1]), as_bf16x8(pb[c][mk][0]), gs[c]);
        if constexpr (P > 1) gs[c] = mfma16x16x32(as_bf16x8(tl.gA[mk][0]), as_bf16x8(pb[c][mk][P - 1]), gs[c]);
      }
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int64_t t = tg + e;
      if (!(colok && t < T)) continue;
      const float4 cf = tl.cf[e];  // pre[t,n], inv[t], scale[t]
      Row o;
#pragma unroll
      for (int w = 0; w < VD; ++w) {
        const uint32_t xw = tl.xr[e][w], gw = tl.gr[e][w];
        const float x0 = __uint_as_float(xw << 16), x1 = __uint_as_float(xw & 0xffff0000u);
        const float g0 = __uint_as_float(gw << 16), g1 = __uint_as_float(gw & 0xffff0000u);
        const float o0 = fmaf(cf.z, x0, fmaf(cf.y, gs[2 * w][e], g0 * cf.x));
        const float o1 = fmaf(cf.z, x1, fmaf(cf.y, gs[2 * w + 1][e], g1 * cf.x));
        o[w] = pack_bf16x2(o0, o1);
      }
      *reinterpret_cast<Row*>(a.gx + (t * N + n) * D + dl) = o;
    }
  };

  const int64_t ntiles = (T + TT - 1) / TT;
  if constexpr (P == 1) {
    Row xn[4], gn[4];  // rows of the next tile
    if (blockIdx.y < ntiles) load_rows(blockIdx.y, xn, gn);
    for (int64_t tile = blockIdx.y; tile < ntiles; tile += a.nsplit) {
      Tile A;
      load_operands(tile, A);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        A.xr[e] = xn[e];
        A.gr[e] = gn[e];
      }
      if (tile + a.nsplit < ntiles) load_rows(tile + a.nsplit, xn, gn);
      compute_tile(tile, A);
    }
  } else {
    for (int64_t tile = blockIdx.y; tile < ntiles; tile += a.nsplit) {
      Tile A;
      load_rows(tile, A.xr, A.gr);
      load_operands(tile, A);
      compute_tile(tile, A);
    }
  }

  if (!colok) return;
  float* part = a.gphi_part + (int64_t)blockIdx.y * M * K;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int m = 16 * mt + 4 * q + v;
      if (m >= M) continue;
#pragma unroll
      for (int c = 0; c < VC; ++c) part[(int64_t)m * K + kcol + c] = ph[mt][c][v];
    }
}

// ---------------------------------------------------------------------------
// Kernel B, LDS-pipelined form (N = 4 / 8, bf16 activations, 16-byte rows)
//
// Same per-lane arithmetic as the streaming form, but the operands of a
// 16-token tile reach the lanes through a ring of S stages in LDS filled by
// direct-to-LDS loads (buffer_load ... lds / global_load_lds): a tile's
// loads are issued S-1 tiles before it is computed and cost no registers
// while in flight, so one block of 4 waves per CU keeps ~(S-1) x 25 KB
// (N = 4) / 32 KB (N = 8) of reads outstanding.  Each direct load moves 16
// bytes per lane to LDS[unit + 16*lane]; a lane later reads back exactly what
// the same lane index loaded, so every LDS read is a conflict-free 16-byte
// row (the coefficients unit excepted: 4 tokens x 4 streams per 64 bytes).
//
// Block (cb, group, split) owns the DW = 128 columns cb*DW.. of the 4
// streams of its group and the tiles split, split + nsplit, ...; blocks of
// one split read
// neighbouring columns of the same token rows at about the same time, which
// measured faster than giving every block an equal contiguous share of the
// (column block, tile) items.
//
// Synchronisation per tile j (slot j % S):
//   wait until this wave's loads of tile j have landed (s_waitcnt vmcnt;
//   vector memory operations complete in issue order), s_barrier, read the
//   tile's operands from LDS, issue the loads of tile j + S - 1 into the
//   slot of tile j - 1 (every wave finished reading it before the barrier),
//   compute, store grad_x with range-checked buffer stores (exactly 4 per
//   lane and tile, so the vmcnt arithmetic is exact).
// Rows of tokens >= T and columns >= D load as zero (range-checked buffer
// loads); grad_mixes rows and coefficients of tokens >= T load from the
// clamped last token and only reach outputs that are not stored.
// ---------------------------------------------------------------------------
// A block owns G = 4 streams (a wave each): N = 8 runs two stream groups
// per column block (blockIdx.x = cb * NG + group), which keeps the phi^T
// operands (VC x MK x P registers) and grad_phi accumulators (MT x VC) of a
// wave within one wave per SIMD.
// With H = 2 (N = 8, one phi plane, no grad_x_in) a stream has two waves,
// one per 64-column half of the block's columns: lane (r, q) of half h
// computes the 4 columns 64h + 4r.. of its tokens (8-byte LDS reads of the
// 16-byte units, which the loads still fill 8 columns a lane), so the
// accumulators and phi^T operands halve (80 + 48 registers) and two waves
// share each SIMD: one wave's LDS, MFMA and barrier waits overlap the
// other's work.  Each wave issues 2 of its stream's 4 x loads and 2 of the
// shared units, 4 loads a tile like every wave of the H = 1 form.
template <int N> struct DmaCfg {
  using PD = PreDims<N>;
  static constexpr int G = 4, NG = N / G;
  static constexpr int VC = 8, VD = 4, DW = 128, TT = 16;
  static constexpr int MK = PD::MK, MT = PD::MT;
  // 1 KB units of one stage (16 bytes per lane)
  static constexpr int X = 0;              // [G][4]  x rows: stream G*group + w, tokens 4q+e
  static constexpr int GY = X + 4 * G;     // [4]     grad_y rows, tokens 4q+e
  static constexpr int GA = GY + 4;        // [MK][2] grad_mixes rows (A of gs), hi/lo
  static constexpr int GT = GA + 2 * MK;   // [MT]    g^T blocks (A of grad_phi), both planes
  static constexpr int CF = GT + MT;       // [1]     coefficients of 16 tokens x G streams
  static constexpr int UNITS = CF + 1;
  static constexpr int GI = UNITS;               // [G][4]  grad_x_in rows (accumulating form)
  static constexpr int UNITS_ACC = GI + 4 * G;
  static constexpr int SHARED = UNITS - GY;      // units loaded once per block, split over waves
  static constexpr int LMIN = 4 + SHARED / G;    // fewest loads a wave issues per tile
  static constexpr int RA = (2 * MK + MT + 3) / 4 * 4;  // units from GA read per tile (4 at a time)
  static constexpr int STAGES = N == 4 ? 5 : 4;  // ring: 125 KB (N = 4) / 128 KB (N = 8) of LDS
  static_assert(N % G == 0 && GA + RA <= UNITS, "stream groups; reads stay in the slot");
};

constexpr int kDmaAccStages = 3;               // accumulating form: 3 x 41 KB (N = 4) / 48 KB (N = 8)
// Only N = 8 runs the two-waves-per-stream (column halves) form.  At N = 4 it
// measured 5-12% faster in a back-to-back timing loop at T <= 32768, where
// part of x stays in the MALL between calls, but 3-4% slower in bench.py,
// which evicts the caches before every call (D = 4096, T = 16384: 342-344
// against 329-333 us), and 4-6% slower at T = 65536 either way.
constexpr int kDmaMaxBlocks = 512;             // bounds the token splits of small D

struct PreBwdDmaArgs {
  const bf16_t* x;
  const bf16_t* gy;
  const uint16_t* phiT;  // [P][K][MP32]
  int64_t phiT_plane_stride;
  const uint16_t* gmP;   // [2][T][MP32]
  int64_t gmP_plane;
  const uint16_t* gTw;   // [ceil(T/16)][MT][64][2][4]
  const float4* coef;    // (T, N) {pre, inv, scale, 0}
  bf16_t* gx;
  const bf16_t* gin;     // accumulating form: grad_x = gin + dL/dx (same layout as x)
  float* part;           // [nsplit][M][K] grad_phi partials
  int64_t T;
  int D;
  int64_t ntiles;
};

// A tile's ring reads, all issued before one wait: with one wave per SIMD the
// LDS latency is then paid once a tile instead of once per group of four
// reads (the groups used to wait in turn).
//   xr[e]    = unit X + 4w + e      (xa: the lane's address of unit X + 4w)
//   gr[e]    = unit GY + e          (la: the lane's address of unit 0)
//   ag[i][e] = unit GA + 4i + e
//   cf[e]    = 16 bytes at cfa + 64e
// The unit offsets are literals: GY = 16, GA = 20 and G = 4 for N = 4 and 8.
template <int RQ>
__device__ __forceinline__ void dma_tile_reads(u32x4 (&xr)[4], u32x4 (&gr)[4], u32x4 (&ag)[RQ][4],
                                               u32x4 (&cf)[4], uint32_t xa, uint32_t la, uint32_t cfa) {
  static_assert(DmaCfg<4>::X == 0 && DmaCfg<4>::GY == 16 && DmaCfg<4>::GA == 20 && DmaCfg<4>::G == 4 &&
                    DmaCfg<8>::X == 0 && DmaCfg<8>::GY == 16 && DmaCfg<8>::GA == 20 && DmaCfg<8>::G == 4,
                "unit offsets written into the reads below");
  static_assert(RQ == 1 || RQ == 3, "read groups of N = 4 / N = 8");
  if constexpr (RQ == 1) {
    asm volatile(
        "ds_read_b128 %0, %16\n\t"
        "ds_read_b128 %1, %16 offset:1024\n\t"
        "ds_read_b128 %2, %16 offset:2048\n\t"
        "ds_read_b128 %3, %16 offset:3072\n\t"
        "ds_read_b128 %4, %17 offset:16384\n\t"
        "ds_read_b128 %5, %17 offset:17408\n\t"
        "ds_read_b128 %6, %17 offset:18432\n\t"
        "ds_read_b128 %7, %17 offset:19456\n\t"
        "ds_read_b128 %8, %17 offset:20480\n\t"
        "ds_read_b128 %9, %17 offset:21504\n\t"
        "ds_read_b128 %10, %17 offset:22528\n\t"
        "ds_read_b128 %11, %17 offset:23552\n\t"
        "ds_read_b128 %12, %18\n\t"
        "ds_read_b128 %13, %18 offset:64\n\t"
        "ds_read_b128 %14, %18 offset:128\n\t"
        "ds_read_b128 %15, %18 offset:192\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(xr[0]), "=&v"(xr[1]), "=&v"(xr[2]), "=&v"(xr[3]), "=&v"(gr[0]), "=&v"(gr[1]), "=&v"(gr[2]),
          "=&v"(gr[3]), "=&v"(ag[0][0]), "=&v"(ag[0][1]), "=&v"(ag[0][2]), "=&v"(ag[0][3]), "=&v"(cf[0]),
          "=&v"(cf[1]), "=&v"(cf[2]), "=&v"(cf[3])
        : "v"(xa), "v"(la), "v"(cfa)
        : "memory");
  } else {
    asm volatile(
        "ds_read_b128 %0, %24\n\t"
        "ds_read_b128 %1, %24 offset:1024\n\t"
        "ds_read_b128 %2, %24 offset:2048\n\t"
        "ds_read_b128 %3, %24 offset:3072\n\t"
        "ds_read_b128 %4, %25 offset:16384\n\t"
        "ds_read_b128 %5, %25 offset:17408\n\t"
        "ds_read_b128 %6, %25 offset:18432\n\t"
        "ds_read_b128 %7, %25 offset:19456\n\t"
        "ds_read_b128 %8, %25 offset:20480\n\t"
        "ds_read_b128 %9, %25 offset:21504\n\t"
        "ds_read_b128 %10, %25 offset:22528\n\t"
        "ds_read_b128 %11, %25 offset:23552\n\t"
        "ds_read_b128 %12, %25 offset:24576\n\t"
        "ds_read_b128 %13, %25 offset:25600\n\t"
        "ds_read_b128 %14, %25 offset:26624\n\t"
        "ds_read_b128 %15, %25 offset:27648\n\t"
        "ds_read_b128 %16, %25 offset:28672\n\t"
        "ds_read_b128 %17, %25 offset:29696\n\t"
        "ds_read_b128 %18, %25 offset:30720\n\t"
        "ds_read_b128 %19, %25 offset:31744\n\t"
        "ds_read_b128 %20, %26\n\t"
        "ds_read_b128 %21, %26 offset:64\n\t"
        "ds_read_b128 %22, %26 offset:128\n\t"
        "ds_read_b128 %23, %26 offset:192\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(xr[0]), "=&v"(xr[1]), "=&v"(xr[2]), "=&v"(xr[3]), "=&v"(gr[0]), "=&v"(gr[1]), "=&v"(gr[2]),
          "=&v"(gr[3]), "=&v"(ag[0][0]), "=&v"(ag[0][1]), "=&v"(ag[0][2]), "=&v"(ag[0][3]), "=&v"(ag[1][0]),
          "=&v"(ag[1][1]), "=&v"(ag[1][2]), "=&v"(ag[1][3]), "=&v"(ag[2][0]), "=&v"(ag[2][1]), "=&v"(ag[2][2]),
          "=&v"(ag[2][3]), "=&v"(cf[0]), "=&v"(cf[1]), "=&v"(cf[2]), "=&v"(cf[3])
        : "v"(xa), "v"(la), "v"(cfa)
        : "memory");
  }
}

// The same reads for H = 2: xr / gr are the 8 bytes of the lane's 4 columns
// (xa, lx: their addresses in unit X + 4w and unit 0), ag / cf as above (la).
template <int RQ>
__device__ __forceinline__ void dma_tile_reads_h2(u32x2 (&xr)[4], u32x2 (&gr)[4], u32x4 (&ag)[RQ][4],
                                                  u32x4 (&cf)[4], uint32_t xa, uint32_t lx, uint32_t la,
                                                  uint32_t cfa) {
  static_assert(RQ == 1 || RQ == 3, "read groups of N = 4 / N = 8");
  if constexpr (RQ == 1) {
    asm volatile(
        "ds_read_b64 %0, %16\n\t"
        "ds_read_b64 %1, %16 offset:1024\n\t"
        "ds_read_b64 %2, %16 offset:2048\n\t"
        "ds_read_b64 %3, %16 offset:3072\n\t"
        "ds_read_b64 %4, %17 offset:16384\n\t"
        "ds_read_b64 %5, %17 offset:17408\n\t"
        "ds_read_b64 %6, %17 offset:18432\n\t"
        "ds_read_b64 %7, %17 offset:19456\n\t"
        "ds_read_b128 %8, %18 offset:20480\n\t"
        "ds_read_b128 %9, %18 offset:21504\n\t"
        "ds_read_b128 %10, %18 offset:22528\n\t"
        "ds_read_b128 %11, %18 offset:23552\n\t"
        "ds_read_b128 %12, %19\n\t"
        "ds_read_b128 %13, %19 offset:64\n\t"
        "ds_read_b128 %14, %19 offset:128\n\t"
        "ds_read_b128 %15, %19 offset:192\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(xr[0]), "=&v"(xr[1]), "=&v"(xr[2]), "=&v"(xr[3]), "=&v"(gr[0]), "=&v"(gr[1]), "=&v"(gr[2]),
          "=&v"(gr[3]), "=&v"(ag[0][0]), "=&v"(ag[0][1]), "=&v"(ag[0][2]), "=&v"(ag[0][3]), "=&v"(cf[0]),
          "=&v"(cf[1]), "=&v"(cf[2]), "=&v"(cf[3])
        : "v"(xa), "v"(lx), "v"(la), "v"(cfa)
        : "memory");
  } else {
    asm volatile(
        "ds_read_b64 %0, %24\n\t"
        "ds_read_b64 %1, %24 offset:1024\n\t"
        "ds_read_b64 %2, %24 offset:2048\n\t"
        "ds_read_b64 %3, %24 offset:3072\n\t"
        "ds_read_b64 %4, %25 offset:16384\n\t"
        "ds_read_b64 %5, %25 offset:17408\n\t"
        "ds_read_b64 %6, %25 offset:18432\n\t"
        "ds_read_b64 %7, %25 offset:19456\n\t"
        "ds_read_b128 %8, %26 offset:20480\n\t"
        "ds_read_b128 %9, %26 offset:21504\n\t"
        "ds_read_b128 %10, %26 offset:22528\n\t"
        "ds_read_b128 %11, %26 offset:23552\n\t"
        "ds_read_b128 %12, %26 offset:24576\n\t"
        "ds_read_b128 %13, %26 offset:25600\n\t"
        "ds_read_b128 %14, %26 offset:26624\n\t"
        "ds_read_b128 %15, %26 offset:27648\n\t"
        "ds_read_b128 %16, %26 offset:28672\n\t"
        "ds_read_b128 %17, %26 offset:29696\n\t"
        "ds_read_b128 %18, %26 offset:30720\n\t"
        "ds_read_b128 %19, %26 offset:31744\n\t"
        "ds_read_b128 %20, %27\n\t"
        "ds_read_b128 %21, %27 offset:64\n\t"
        "ds_read_b128 %22, %27 offset:128\n\t"
        "ds_read_b128 %23, %27 offset:192\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(xr[0]), "=&v"(xr[1]), "=&v"(xr[2]), "=&v"(xr[3]), "=&v"(gr[0]), "=&v"(gr[1]), "=&v"(gr[2]),
          "=&v"(gr[3]), "=&v"(ag[0][0]), "=&v"(ag[0][1]), "=&v"(ag[0][2]), "=&v"(ag[0][3]), "=&v"(ag[1][0]),
          "=&v"(ag[1][1]), "=&v"(ag[1][2]), "=&v"(ag[1][3]), "=&v"(ag[2][0]), "=&v"(ag[2][1]), "=&v"(ag[2][2]),
          "=&v"(ag[2][3]), "=&v"(cf[0]), "=&v"(cf[1]), "=&v"(cf[2]), "=&v"(cf[3])
        : "v"(xa), "v"(lx), "v"(la), "v"(cfa)
        : "memory");
  }
}

template <int N, int P, int S, bool ACC, int H = 1>
__global__ __launch_bounds__(64 * DmaCfg<N>::G * H) void pre_bwd_dma_kernel(PreBwdDmaArgs a) {
  using C = DmaCfg<N>;
  using PD = PreDims<N>;
  constexpr int M = PD::M, MT = PD::MT, MK = PD::MK, MP32 = PD::MP32;
  constexpr int VC = C::VC / H, VD = C::VD / H, DW = C::DW, TT = C::TT;
  constexpr int UNITS = ACC ? C::UNITS_ACC : C::UNITS;
  static_assert(H == 1 || (H == 2 && P == 1 && !ACC), "column halves: one phi plane, no grad_x_in");
  constexpr int XL = 4 / H;                                  // x loads of a wave per tile
  constexpr int LMIN = XL + C::SHARED / (C::G * H) + (ACC ? 4 : 0);  // grad_x_in: 4 more loads a wave
  constexpr int VM_START = (S - 2) * LMIN;                  // before any grad_x store
  constexpr int VM_STEADY = (S - 2) * LMIN + (S - 1) * 4;
  static_assert(S >= 2 && VM_STEADY < 64, "pipeline shape");
  __shared__ u32x4 ring[S * UNITS * kWave];

  const int lane = threadIdx.x & (kWave - 1);
  const int wid = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int w = wid % C::G, h = wid / C::G;  // stream of the group, column half
  const int grp = (int)(blockIdx.x % C::NG), cb = (int)(blockIdx.x / C::NG);
  const int n = grp * C::G + w;
  const int r = lane & 15, q = lane >> 4;
  const int D = a.D;
  const int64_t T = a.T, K = (int64_t)N * D, ntiles = a.ntiles;
  const int64_t tstep = gridDim.y;
  const int64_t cnt = (ntiles - blockIdx.y + tstep - 1) / tstep;
  if (cnt <= 0) return;  // uniform over the block
  const int dl = cb * DW + (DW / H) * h + VC * r;  // first column this lane computes
  const bool colok = dl < D;
  const int dld = cb * DW + 8 * r;  // first column this lane's 16-byte loads move
  const bool ldok = dld < D;

  int64_t itile = blockIdx.y;  // next tile to load
  auto issue = [&](int64_t j) {
    const int64_t tile = itile, tb = tile * TT;
    itile += tstep;
    const int nv = (int)(T - tb < TT ? T - tb : TT);
    u32x4* st = ring + (int)(j % S) * UNITS * kWave;
    const auto rx = rows_rsrc(a.x + tb * K, (int64_t)nv * K * 2);
#pragma unroll
    for (int e = XL * h; e < XL * h + XL; ++e) {
      const uint32_t off = ldok ? (uint32_t)((((4 * q + e) * N + n) * (int64_t)D + dld) * 2) : kBufferOob;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rx, (lds_void_t*)(st + (C::X + 4 * w + e) * kWave), 16,
                                               off, 0, 0, 2 /* nt */);
    }
    if constexpr (ACC) {
      const auto ri = rows_rsrc(a.gin + tb * K, (int64_t)nv * K * 2);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const uint32_t off = ldok ? (uint32_t)((((4 * q + e) * N + n) * (int64_t)D + dld) * 2) : kBufferOob;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(ri, (lds_void_t*)(st + (C::GI + 4 * w + e) * kWave), 16,
                                                 off, 0, 0, 2 /* nt */);
      }
    }
    for (int u = wid; u < C::SHARED; u += C::G * H) {
      const int unit = C::GY + u;
      lds_void_t* dst = (lds_void_t*)(st + unit * kWave);
      if (unit < C::GA) {
        const int e = unit - C::GY;
        const auto rg = rows_rsrc(a.gy + tb * D, (int64_t)nv * D * 2);
        const uint32_t off = ldok ? (uint32_t)(((4 * q + e) * (int64_t)D + dld) * 2) : kBufferOob;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rg, dst, 16, off, 0, 0, 2);
      } else if (unit < C::GT) {
        const int mk = (unit - C::GA) >> 1, g = (unit - C::GA) & 1;
        const int64_t ts = tb + r < T ? tb + r : T - 1;
        __builtin_amdgcn_global_load_lds((glb_void_t*)(a.gmP + g * a.gmP_plane + ts * MP32 + 32 * mk + 8 * q),
                                         dst, 16, 0, 0);
      } else if (unit < C::CF) {
        const int mt = unit - C::GT;
        __builtin_amdgcn_global_load_lds((glb_void_t*)(a.gTw + ((tile * MT + mt) * kWave + lane) * 8), dst,
                                         16, 0, 0);
      } else {  // token lane / G, stream G * group + lane % G
        int64_t idx = (tb + lane / C::G) * N + grp * C::G + lane % C::G;
        if (idx > T * N - 1) idx = T * N - 1;
        __builtin_amdgcn_global_load_lds((glb_void_t*)(a.coef + idx), dst, 16, 0, 0);
      }
    }
  };

  // phi^T operands of the block's columns and the grad_phi accumulators
  u32x4 pb[VC][MK][P];
  {
    const int64_t kcol = (int64_t)n * D + (colok ? dl : 0);
#pragma unroll
    for (int c = 0; c < VC; ++c)
#pragma unroll
      for (int mk = 0; mk < MK; ++mk)
#pragma unroll
        for (int p = 0; p < P; ++p) {
          const u32x4 v = ld16(a.phiT + p * a.phiT_plane_stride + (kcol + c) * MP32 + 32 * mk + 8 * q);
          pb[c][mk][p] = colok ? v : zero4();
        }
  }
  floatx4 ph[MT][VC];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int c = 0; c < VC; ++c) ph[mt][c] = floatx4{0.f, 0.f, 0.f, 0.f};

  // LDS reads of the ring are inline asm (lds_read4), ordered after the
  // direct-to-LDS loads by the explicit waits.
  const uint32_t ring_lds = lds_addr(ring);

  for (int64_t j = 0; j < S - 1 && j < cnt; ++j) issue(j);

  int64_t ctile = blockIdx.y;
  for (int64_t j = 0; j < cnt; ++j, ctile += tstep) {
    // this wave's loads of tile j have landed once at most V newer vector
    // memory operations are outstanding
    if (j + S - 2 < cnt) {
      if (j >= S - 1)
        wait_vmcnt<VM_STEADY>();
      else
        wait_vmcnt<VM_START>();
    } else {
      wait_vmcnt<0>();
    }
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");

    // the next loads go to the slot of tile j - 1, which every wave
    // finished reading before the barrier
    if (j + S - 1 < cnt) issue(j + S - 1);

    const uint32_t sbase = ring_lds + (uint32_t)((j % S) * UNITS * kWave * 16);
    const uint32_t la = sbase + lane * 16;
    uint32_t xr[4][VD], gr[4][VD];  // the lane's columns of x (stream n) and grad_y, tokens 4q+e
    u32x4 gA[MK][2], gt[MT], cfu[4];
    {
      // x rows of stream n and grad_y rows (tokens 4q+e); units GA.. four at
      // a time: grad_mixes hi, lo per mk, then the g^T blocks; coefficients
      // of tokens 4q+e, stream n
      u32x4 ag[C::RA / 4][4];
      const uint32_t xa = la + (C::X + 4 * w) * 1024, cfa = sbase + C::CF * 1024 + (4 * q * C::G + w) * 16;
      if constexpr (H == 2) {
        // byte 8 * r + 128 * h of the q-th 256 bytes holds columns 64h + 4r..
        const uint32_t lx = sbase + 256 * q + 128 * h + 8 * r;
        u32x2 x2[4], g2[4];
        dma_tile_reads_h2<C::RA / 4>(x2, g2, ag, cfu, lx + (C::X + 4 * w) * 1024, lx, la, cfa);
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
          for (int v = 0; v < VD; ++v) {
            xr[e][v] = x2[e][v];
            gr[e][v] = g2[e][v];
          }
      } else {
        u32x4 x4[4], g4[4];
        if constexpr (N == 8 && P == 2) {  // the single-wait form spills with two phi planes at N = 8
          lds_read4<1024>(x4, xa);
          lds_read4<1024>(g4, la + C::GY * 1024);
#pragma unroll
          for (int i = 0; i < C::RA / 4; ++i) lds_read4<1024>(ag[i], la + (C::GA + 4 * i) * 1024);
          lds_read4<C::G * 16>(cfu, cfa);
        } else {
          dma_tile_reads<C::RA / 4>(x4, g4, ag, cfu, xa, la, cfa);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
          for (int v = 0; v < VD; ++v) {
            xr[e][v] = x4[e][v];
            gr[e][v] = g4[e][v];
          }
      }
#pragma unroll
      for (int mk = 0; mk < MK; ++mk) {
        gA[mk][0] = ag[(2 * mk) / 4][(2 * mk) % 4];
        gA[mk][1] = ag[(2 * mk + 1) / 4][(2 * mk + 1) % 4];
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) gt[mt] = ag[(2 * MK + mt) / 4][(2 * MK + mt) % 4];
    }
    u32x4 gi[4];
    if constexpr (ACC) lds_read4<1024>(gi, la + (C::GI + 4 * w) * 1024);  // grad_x_in rows, tokens 4q+e

    const int64_t tb = ctile * TT;
    const int nv = (int)(T - tb < TT ? T - tb : TT);

    // ---- grad_phi partial += g^T @ x over the tile's 16 tokens ------------
#pragma unroll
    for (int c = 0; c < VC; ++c) {
      u32x2 xt;  // column c of the lane's 4 x VC block: tokens (2w, 2w+1) in dword w
#pragma unroll
      for (int w = 0; w < 2; ++w) {
        const uint32_t lo = xr[2 * w][c >> 1], hi = xr[2 * w + 1][c >> 1];
        xt[w] = (c & 1) ? ((lo >> 16) | (hi & 0xffff0000u)) : ((lo & 0xffffu) | (hi << 16));
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        ph[mt][c] = mfma16x16x16(u32x2{gt[mt][0], gt[mt][1]}, xt, ph[mt][c]);
        ph[mt][c] = mfma16x16x16(u32x2{gt[mt][2], gt[mt][3]}, xt, ph[mt][c]);
      }
    }
    // ---- gs = grad_mixes @ phi, then grad_x ---------------------------------
    floatx4 gs[VC];
#pragma unroll
    for (int c = 0; c < VC; ++c) {
      gs[c] = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int mk = 0; mk < MK; ++mk) {
        gs[c] = mfma16x16x32(as_bf16x8(gA[mk][0]), as_bf16x8(pb[c][mk][0]), gs[c]);
        gs[c] = mfma16x16x32(as_bf16x8(gA[mk][1]), as_bf16x8(pb[c][mk][0]), gs[c]);
        if constexpr (P > 1) gs[c] = mfma16x16x32(as_bf16x8(gA[mk][0]), as_bf16x8(pb[c][mk][P - 1]), gs[c]);
      }
    }
    const auto rgx = rows_rsrc(a.gx + tb * K, (int64_t)nv * K * 2);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      // pre[t,n], inv[t], scale[t]
      const float fx = __uint_as_float(cfu[e][0]), fy = __uint_as_float(cfu[e][1]),
                  fz = __uint_as_float(cfu[e][2]);
      uint32_t o[4] = {0u, 0u, 0u, 0u};
#pragma unroll
      for (int w = 0; w < VD; ++w) {
        const uint32_t xw = xr[e][w], gw = gr[e][w];
        const float x0 = __uint_as_float(xw << 16), x1 = __uint_as_float(xw & 0xffff0000u);
        const float g0 = __uint_as_float(gw << 16), g1 = __uint_as_float(gw & 0xffff0000u);
        float o0 = fmaf(fz, x0, fmaf(fy, gs[2 * w][e], g0 * fx));
        float o1 = fmaf(fz, x1, fmaf(fy, gs[2 * w + 1][e], g1 * fx));
        if constexpr (ACC) {
          o0 += __uint_as_float(gi[e][w] << 16);
          o1 += __uint_as_float(gi[e][w] & 0xffff0000u);
        }
        o[w] = pack_bf16x2(o0, o1);
      }
      // rows >= nv fall outside the range and are dropped, as are columns >= D;
      // streaming (nt) stores measured 6% faster for this kernel than default ones
      const uint32_t off = colok ? (uint32_t)((((4 * q + e) * N + n) * (int64_t)D + dl) * 2) : kBufferOob;
      if constexpr (H == 2)
        __builtin_amdgcn_raw_buffer_store_b64(u32x2{o[0], o[1]}, rgx, off, 0, 2 /* nt */);
      else
        __builtin_amdgcn_raw_buffer_store_b128(u32x4{o[0], o[1], o[2], o[3]}, rgx, off, 0, 2 /* nt */);
    }
  }

  if (!colok) return;
  float* part = a.part + (int64_t)blockIdx.y * M * K + (int64_t)n * D + dl;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int m = 16 * mt + 4 * q + v;
      if (m >= M) continue;
      float4* dst = reinterpret_cast<float4*>(part + (int64_t)m * K);
#pragma unroll
      for (int c4 = 0; c4 < VC / 4; ++c4)
        dst[c4] = float4{ph[mt][4 * c4][v], ph[mt][4 * c4 + 1][v], ph[mt][4 * c4 + 2][v], ph[mt][4 * c4 + 3][v]};
    }
}

// ---------------------------------------------------------------------------
// Kernels C: fixed-order reductions
// ---------------------------------------------------------------------------
__global__ void sum_splits_kernel(const float* __restrict__ part, float* __restrict__ out,
                                  int64_t n, int nsplit) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    float s = 0.f;
    for (int j = 0; j < nsplit; ++j) s += part[(int64_t)j * n + i];
    out[i] = s;
  }
}

// ---------------------------------------------------------------------------
// Compensated grad_phi (opt-in, MHC_PRE_BWD_COMPENSATED)
//
// grad_phi[m,k] = sum_t g[t,m] * x[t,k] with g = grad_mixes * inv_rms (the
// same fp32 product the streaming kernels use).  g is split into three bf16
// planes (exact to 2^-26) and x into 1 (bf16), 2 (fp16, exact) or 3 (fp32)
// planes, so the products on v_mfma_f32_16x16x32_bf16 (32 tokens deep) are
// exact and only their fp32 additions round.  Each wave owns 16 * VC columns
// of one token split and adds every 32-token tile's MFMA result into a
// (sum, compensation) pair per output (Kahan); the splits' sums are added
// with Neumaier's compensation in a fixed order.  Columns of the lane's
// 8-token x VC-column block are transposed in registers into the MFMA B
// operand, as in the streaming kernels; no LDS.
// ---------------------------------------------------------------------------
constexpr int kCompPlanesG = 3;
constexpr int kCompTile = 32;  // tokens per MFMA (K of 16x16x32)

// g planes in MFMA A-operand order: [ceil(T/32)][MT][64 lanes][3 planes][8
// tokens] bf16, lane = m % 16 + 16 * q holding tokens 32 * tile + 8q + j.
template <int N>
__global__ void comp_gplanes_kernel(const float* __restrict__ gm, const float* __restrict__ inv,
                                    uint16_t* __restrict__ gpl, int64_t T, int64_t ntiles) {
  using PD = PreDims<N>;
  constexpr int M = PD::M, MT = PD::MT;
  const int64_t n = ntiles * MT * kWave;
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int lane = (int)(i % kWave);
    const int64_t tm = i / kWave;
    const int mt = (int)(tm % MT);
    const int64_t tile = tm / MT;
    const int m = 16 * mt + (lane & 15);
    uint32_t pl[kCompPlanesG][8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int64_t t = kCompTile * tile + 8 * (lane >> 4) + j;
      float v = (t < T && m < M) ? gm[t * M + m] * inv[t] : 0.f;
#pragma unroll
      for (int p = 0; p < kCompPlanesG; ++p) {
        pl[p][j] = f32_to_bf16_bits(v);
        v -= bf16_bits_to_f32(pl[p][j]);
      }
    }
    u32x4* dst = reinterpret_cast<u32x4*>(gpl + i * (kCompPlanesG * 8));
#pragma unroll
    for (int p = 0; p < kCompPlanesG; ++p) {
      u32x4 v;
#pragma unroll
      for (int w = 0; w < 4; ++w) v[w] = pl[p][2 * w] | (pl[p][2 * w + 1] << 16);
      dst[p] = v;
    }
  }
}

struct GphiCompArgs {
  const void* x;         // (T, K) activations
  const uint16_t* gpl;   // g planes, layout above
  float* part;           // [2][nsplit][M][K]: sums, then compensations
  int64_t T, K, tps;     // tps: tokens per split, a multiple of kCompTile
  int nsplit;
};

template <typename S> struct XPlanes { static constexpr int P = 3; };                     // fp32
template <> struct XPlanes<bf16_t> { static constexpr int P = 1; };
template <> struct XPlanes<f16_t> { static constexpr int P = 2; };

// Raw bits of VC consecutive elements of `row` from column k (zeros past K or
// when !ok), as NW = VC * sizeof(S) / 4 words (2-byte types two per word, low
// half first).  Kept raw so that the loads of the next tile stay in flight
// while the current one is multiplied.
template <typename S, int VC> struct XRaw {
  static constexpr int NW = VC * (int)sizeof(S) / 4;
};

template <typename S, int VC, bool VEC>
__device__ __forceinline__ void load_raw(const S* row, int64_t k, int64_t K, bool ok, uint32_t* w) {
  constexpr int NW = XRaw<S, VC>::NW;
  if constexpr (VEC) {
    // K % VC == 0 and 16-byte aligned rows: the group is wholly in or out
    const bool in = ok && k < K;
    if constexpr (NW == 2) {
      const uint2 v = in ? *reinterpret_cast<const uint2*>(row + k) : uint2{0u, 0u};
      w[0] = v.x;
      w[1] = v.y;
    } else {
      static_assert(NW % 4 == 0, "16-byte groups");
#pragma unroll
      for (int i = 0; i < NW / 4; ++i) {
        const u32x4 v = in ? ld16nt(reinterpret_cast<const char*>(row + k) + 16 * i) : zero4();
#pragma unroll
        for (int j = 0; j < 4; ++j) w[4 * i + j] = v[j];
      }
    }
  } else if constexpr (sizeof(S) == 2) {
    const uint16_t* r16 = reinterpret_cast<const uint16_t*>(row);
#pragma unroll
    for (int i = 0; i < NW; ++i) {
      const uint32_t lo = (ok && k + 2 * i < K) ? r16[k + 2 * i] : 0u;
      const uint32_t hi = (ok && k + 2 * i + 1 < K) ? r16[k + 2 * i + 1] : 0u;
      w[i] = lo | (hi << 16);
    }
  } else {
#pragma unroll
    for (int i = 0; i < NW; ++i) w[i] = (ok && k + i < K) ? __float_as_uint(row[k + i]) : 0u;
  }
}

// bf16 planes of element i of a raw group
template <typename S, int PX>
__device__ __forceinline__ void raw_planes(const uint32_t* w, int i, uint32_t* pl) {
  if constexpr (std::is_same<S, bf16_t>::value) {
    pl[0] = (w[i >> 1] >> (16 * (i & 1))) & 0xffffu;
  } else {
    float v;
    if constexpr (sizeof(S) == 4)
      v = __uint_as_float(w[i]);
    else
      v = Store<S>::to_f32((uint16_t)((w[i >> 1] >> (16 * (i & 1))) & 0xffffu));
#pragma unroll
    for (int p = 0; p < PX; ++p) {
      pl[p] = f32_to_bf16_bits(v);
      if (p + 1 < PX) v -= bf16_bits_to_f32(pl[p]);
    }
  }
}

template <int N, typename S, int VC, bool VEC>
__global__ __launch_bounds__(kWave) void pre_bwd_gphi_comp_kernel(GphiCompArgs a) {
  using PD = PreDims<N>;
  constexpr int M = PD::M, MT = PD::MT, PX = XPlanes<S>::P, PG = kCompPlanesG, NW = XRaw<S, VC>::NW;
  const int lane = threadIdx.x, r = lane & 15, q = lane >> 4;
  const S* __restrict__ x = static_cast<const S*>(a.x);
  const int64_t T = a.T, K = a.K;
  const int64_t kl = (int64_t)blockIdx.x * (16 * VC) + (int64_t)VC * r;  // lane's first column
  const int64_t tb0 = (int64_t)blockIdx.y * a.tps;
  const int64_t tb1 = tb0 + a.tps < T ? tb0 + a.tps : T;

  floatx4 sum[MT][VC], cmp[MT][VC];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int c = 0; c < VC; ++c) sum[mt][c] = cmp[mt][c] = floatx4{0.f, 0.f, 0.f, 0.f};

  // operands of 32-token tiles: g planes (A) and this lane's x rows (tokens
  // tb + 8q + e, columns kl .. kl + VC - 1), in NS slots loaded NS tiles
  // ahead of the one being multiplied (two slots measured no faster and
  // cost registers)
  constexpr int TT = kCompTile, NS = 1;
  uint32_t xw[NS][8][NW];
  u32x4 ga[NS][MT][PG];
  auto load_tile = [&](int64_t tb, int slot) {
    const u32x4* gp = reinterpret_cast<const u32x4*>(a.gpl) + ((tb / TT) * MT * kWave + lane) * PG;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int p = 0; p < PG; ++p) ga[slot][mt][p] = gp[mt * kWave * PG + p];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int64_t t = tb + 8 * q + e;
      const bool ok = t < T;
      load_raw<S, VC, VEC>(x + (ok ? t : 0) * K, kl, K, ok, xw[slot][e]);
    }
  };
  auto multiply = [&](const uint32_t (&cw)[8][NW], const u32x4 (&cg)[MT][PG]) {
#pragma unroll
    for (int c = 0; c < VC; ++c) {
      u32x4 xb[PX];
      if constexpr (std::is_same<S, bf16_t>::value) {
        // column c of tokens (2w, 2w + 1) straight from the raw words
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const uint32_t lo = cw[2 * w][c >> 1], hi = cw[2 * w + 1][c >> 1];
          xb[0][w] = (c & 1) ? ((lo >> 16) | (hi & 0xffff0000u)) : ((lo & 0xffffu) | (hi << 16));
        }
      } else {
        uint32_t pl[8][PX];
#pragma unroll
        for (int e = 0; e < 8; ++e) raw_planes<S, PX>(cw[e], c, pl[e]);
#pragma unroll
        for (int p = 0; p < PX; ++p)
#pragma unroll
          for (int w = 0; w < 4; ++w) xb[p][w] = pl[2 * w][p] | (pl[2 * w + 1][p] << 16);
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        floatx4 tile = floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int pg = 0; pg < PG; ++pg)
#pragma unroll
          for (int px = 0; px < PX; ++px)
            if (pg + px <= 3) tile = mfma16x16x32(as_bf16x8(cg[mt][pg]), as_bf16x8(xb[px]), tile);
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          float sv = sum[mt][c][v], cv = cmp[mt][c][v];
          kahan_add(sv, cv, tile[v]);
          sum[mt][c][v] = sv;
          cmp[mt][c][v] = cv;
        }
      }
    }
  };
  // tile tb + j * TT lives in slot j % NS; a slot is refilled (NS tiles
  // ahead) right after its contents are copied out
  auto step = [&](int64_t tb, int slot) {
    uint32_t cw[8][NW];
    u32x4 cg[MT][PG];
#pragma unroll
    for (int e = 0; e < 8; ++e)
#pragma unroll
      for (int i = 0; i < NW; ++i) cw[e][i] = xw[slot][e][i];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int p = 0; p < PG; ++p) cg[mt][p] = ga[slot][mt][p];
    if (tb + NS * TT < tb1) load_tile(tb + NS * TT, slot);
    multiply(cw, cg);
  };

#pragma unroll
  for (int j = 0; j < NS; ++j)
    if (tb0 + j * TT < tb1) load_tile(tb0 + j * TT, j);
  for (int64_t tb = tb0; tb < tb1; tb += NS * TT) {
#pragma unroll
    for (int j = 0; j < NS; ++j)
      if (tb + j * TT < tb1) step(tb + j * TT, j);
  }

  const int64_t MK = (int64_t)M * K;
  float* ps = a.part + (int64_t)blockIdx.y * MK;
  float* pc = a.part + ((int64_t)a.nsplit + blockIdx.y) * MK;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const int m = 16 * mt + 4 * q + v;
      if (m >= M) continue;
#pragma unroll
      for (int c = 0; c < VC; ++c) {
        if (kl + c >= K) continue;
        ps[(int64_t)m * K + kl + c] = sum[mt][c][v];
        pc[(int64_t)m * K + kl + c] = -cmp[mt][c][v];  // Kahan's c is the negated error
      }
    }
}

// out[i] = compensated sum over the splits of sums[j][i], plus their
// compensations
__global__ void sum_splits_comp_kernel(const float* __restrict__ part, float* __restrict__ out, int64_t n,
                                       int nsplit) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x) {
    float s = 0.f, c = 0.f;
    for (int j = 0; j < nsplit; ++j) {
      neumaier_add(s, c, part[(int64_t)j * n + i]);
      c += part[((int64_t)nsplit + j) * n + i];
    }
    out[i] = s + c;
  }
}

// One block per column c of partial (rows x C): out = sum over rows.
// comp: each thread sums its rows with Neumaier's compensation, then the 256
// (sum, compensation) pairs are added pairwise with the exact error of each
// addition (TwoSum) carried into the compensation.
// status (may be null): the single-pass kernel's status word; nonzero (a
// timed-out wait) makes the outputs NaN.
__global__ __launch_bounds__(256) void sum_rows_kernel(const float* __restrict__ partial,
                                                       int64_t rows, int C,
                                                       float* __restrict__ out_alpha,
                                                       float* __restrict__ out_base, int comp,
                                                       const uint32_t* status) {
  __shared__ float red[256], redc[256];
  const int c = blockIdx.x;
  float s = 0.f, cc = 0.f;
  if (comp) {
    for (int64_t i = threadIdx.x; i < rows; i += 256) neumaier_add(s, cc, partial[i * C + c]);
  } else {
    for (int64_t i = threadIdx.x; i < rows; i += 256) s += partial[i * C + c];
  }
  red[threadIdx.x] = s;
  redc[threadIdx.x] = cc;
  __syncthreads();
  for (int w = 128; w > 0; w >>= 1) {
    if ((int)threadIdx.x < w) {
      const float a0 = red[threadIdx.x], b0 = red[threadIdx.x + w];
      const float t = a0 + b0;
      if (comp) {
        const float bb = t - a0;
        redc[threadIdx.x] += redc[threadIdx.x + w] + ((a0 - (t - bb)) + (b0 - bb));
      }
      red[threadIdx.x] = t;
    }
    __syncthreads();
  }
  if (threadIdx.x == 0 && comp) red[0] += redc[0];
  if (threadIdx.x == 0 && status && *status) red[0] = __builtin_nanf("");
  if (threadIdx.x == 0) {
    if (c < 3)
      out_alpha[c] = red[0];
    else
      out_base[c - 3] = red[0];
  }
}

}  // namespace mhc

#include "pre_bwd_coop.hpp"

namespace mhc {

__global__ void zero_kernel(float* p, int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    p[i] = 0.f;
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
struct BwdLayout {
  int M, L, C, P, MP, MP32, nsplit, chunks, DC, gpre_chunks;
  int64_t K, nblkA, tok_per_split, ntiles;
  size_t off_phiT, off_gm, off_scale, off_partial, off_gphi, off_sink, off_gpre, off_gpl;
  size_t off_gmP, off_gTw, off_coef, total;
  // single-pass form (0 when it cannot apply): G members per group, control
  // words + exchange ring, contribution rows after kernel A's
  int bcG, bcMaxg;
  int64_t bc_rows;
  size_t off_bc_ctl, bc_ring_bytes;
};

// The single-pass backward: N = 4, bf16 phi, a slice geometry for D and
// at least kBcMinT tokens (below it the two-pass forms' grid fills the chip
// better), kBcAutoT without a pass flag.  Measured on MI355X (bf16, D = 7168
// unless noted, backward ms, single / two-pass): T = 8192 0.294 / 0.307, T =
// 16384 0.526 / 0.587, T = 16384 at D = 4096 0.294 / 0.341, T = 32768 0.987 /
// 1.192, T = 65536 1.92 / 2.42.
constexpr int64_t kBcMinT = 8192, kBcAutoT = 8192;
inline bool bc_shape(int64_t T, int N, int D, int32_t phi_dtype, int* G) {
  return N == 4 && phi_dtype == MHC_DTYPE_BF16 && T >= kBcMinT && coop_nch(D, G);
}

// Token splits of the grad_phi partials: kMaxSplits for the split kernels,
// more for the LDS-pipelined kernel when D has few 128-column blocks.
// Below kGpreSplitMaxT tokens grad_pre comes from the split kernel: kernel
// A's grid (a block per 16 tokens) leaves the chip partly idle (measured on
// MI355X at D = 7168, eager calls: T = 64 113 -> 52 us, T = 4096 214 -> 170
// us for the whole backward; even at 16384, 3% slower at 65536).  At T <= 4
// the GPU time still drops (28.0 -> 24.9 us from graph replays) while an
// eager call pays about 2 us more host time for the extra launch.
constexpr int64_t kGpreSplitMinT = 1, kGpreSplitMaxT = 16384;
// From this many tokens bf16 rows take the LDS-pipelined grad_pre kernel
// (a wave per token, so it needs many tokens to fill the chip).
constexpr int64_t kGpreDmaMinT = 16384;

static int64_t dma_max_splits(int D) {
  const int64_t ncb = (D + DmaCfg<4>::DW - 1) / DmaCfg<4>::DW;
  const int64_t s = kDmaMaxBlocks / ncb;
  return s > kMaxSplits ? s : kMaxSplits;
}

// Workspace layout.  It covers both forms of kernel B (the streaming one for
// bf16 activations and the LDS-staged one for the other dtypes / unaligned
// rows), so the size depends only on (T, N, D, phi dtype, iterations).
static BwdLayout bwd_layout(int64_t T, int N, int D, int32_t phi_dtype, int iters) {
  BwdLayout b{};
  b.M = 2 * N + N * N;
  b.L = N * N;
  b.C = 3 + b.M;
  b.P = phi_bwd_planes(phi_dtype);
  b.MP = (int)round_up(b.M, 16);
  b.MP32 = (int)round_up(b.M, 32);
  b.K = (int64_t)N * D;
  b.DC = kMainKC / N;
  b.chunks = (int)((D + b.DC - 1) / b.DC);
  b.nblkA = (T + kBwdTile - 1) / kBwdTile;
  b.ntiles = (T + kStreamTile - 1) / kStreamTile;
  int ns = (1024 + b.chunks - 1) / b.chunks;
  if (ns > kMaxSplits) ns = kMaxSplits;
  const int64_t max_by_t = (T + kMainTS - 1) / kMainTS;
  if (ns > max_by_t) ns = (int)max_by_t;
  if (ns < 1) ns = 1;
  b.tok_per_split = round_up((T + ns - 1) / ns, kMainTS);
  if (b.tok_per_split < kMainTS) b.tok_per_split = kMainTS;
  b.nsplit = (int)((T + b.tok_per_split - 1) / b.tok_per_split);
  if (b.nsplit < 1) b.nsplit = 1;
  size_t off = 0;
  b.off_phiT = off;
  off += align256(phiT_planes_bytes(phi_dtype, b.M, b.K));
  b.off_gm = off;
  off += align256((size_t)T * b.M * 4);
  b.off_scale = off;
  off += align256((size_t)T * 4);
  b.bcG = 0;
  if (bc_shape(T, N, D, phi_dtype, &b.bcG)) {
    b.bcMaxg = coop_max_groups(b.bcG);
    b.bc_rows = device_cu_count();
  } else {
    b.bcG = b.bcMaxg = 0;
    b.bc_rows = 0;
  }
  b.off_partial = off;
  off += align256((size_t)(b.nblkA + b.bc_rows) * b.C * 4);
  b.off_gphi = off;
  off += align256((size_t)dma_max_splits(D) * b.M * b.K * 4);  // grad_phi split partials
  b.off_gmP = off;
  off += align256((size_t)2 * T * b.MP32 * 2);
  b.off_gTw = off;
  off += align256((size_t)b.ntiles * 2 * b.MP * kStreamTile * 2);
  b.off_coef = off;
  off += align256((size_t)T * N * 16);
  b.off_sink = off;
  if (iters > kSinkRegIters) off += align256((size_t)(iters - 1) * b.nblkA * kBwdTile * b.L * 4);
  // N = 8: the split kernel at every T (the backward at D = 2048 / 7168 /
  // 4096, T = 32768 / 16384 / 65536: 0.8% / 1.7% / 0.5% faster than kernel
  // A's own wave-per-token grad_pre loop)
  const int64_t max_t = N == 8 ? INT64_MAX : kGpreSplitMaxT;
  b.gpre_chunks = (T >= kGpreSplitMinT && T < max_t) ? (int)((D + kGpreCols - 1) / kGpreCols) : 0;
  b.off_gpre = off;  // at least one chunk: the LDS-pipelined grad_pre kernel's sums
  off += align256((size_t)T * (b.gpre_chunks > 0 ? b.gpre_chunks : 1) * N * 4);
  b.off_gpl = off;  // compensated mode: g planes, 3 bf16 per (token, padded m)
  off += align256((size_t)((T + kCompTile - 1) / kCompTile) * kCompTile * b.MP * kCompPlanesG * 2);
  b.off_bc_ctl = off;  // control words, then the exchange ring (contiguous: zeroed together)
  b.bc_ring_bytes = b.bcG ? (size_t)b.bcMaxg * kBcR * b.bcG * kBcRecWords * 16 : 0;
  if (b.bcG) off += align256((size_t)kCoCtlWords * 4) + align256(b.bc_ring_bytes);
  b.total = off;
  return b;
}

template <int N, int P>
static int stream_blocks_per_cu() {
  static std::atomic<int> cache{0};
  int nb = cache.load(std::memory_order_relaxed);
  if (nb > 0) return nb;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, pre_bwd_stream_kernel<N, P>, 64 * N, 0) != hipSuccess || nb <= 0)
    nb = 1;
  cache.store(nb, std::memory_order_relaxed);
  return nb;
}

template <int N, int P>
static int launch_stream(const BwdLayout& lay, PreBwdStreamArgs& sta, hipStream_t st) {
  constexpr int DW = StreamCfg<N>::DW;
  const int chunks = (int)((lay.K / N + DW - 1) / DW);
  int64_t ns = (int64_t)device_cu_count() * stream_blocks_per_cu<N, P>() / chunks;
  if (ns > kMaxSplits) ns = kMaxSplits;
  if (ns > lay.ntiles) ns = lay.ntiles;
  if (ns < 1) ns = 1;
  sta.nsplit = (int)ns;
  hipLaunchKernelGGL((pre_bwd_stream_kernel<N, P>), dim3((unsigned)chunks, (unsigned)ns),
                     dim3(64 * N), 0, st, sta);
  return check_launch("pre_bwd_stream");
}

static unsigned reduce_grid(int64_t n) {
  int64_t g = (n + 255) / 256;
  return (unsigned)(g > 8192 ? 8192 : g);
}

static int sum_alpha_base(const BwdLayout& lay, const PreBwdSmallArgs& sa, float* grad_alpha,
                          float* grad_base, hipStream_t st, int64_t extra_rows = 0,
                          const uint32_t* status = nullptr) {
  hipLaunchKernelGGL(sum_rows_kernel, dim3((unsigned)lay.C), dim3(256), 0, st, sa.partial,
                     lay.nblkA + extra_rows, lay.C, grad_alpha, grad_base, sa.comp, status);
  return check_launch("pre_bwd_sum_rows");
}

// Compensated grad_phi: g planes, then the split MFMA sums, then their
// compensated fixed-order sum.  Reuses the grad_phi partial region (the plain
// partials written there before are not read in this mode).
template <int N, typename S, int VC, bool VEC>
static int launch_comp_gphi_v(const BwdLayout& lay, const GphiCompArgs& ga, int64_t ncw, hipStream_t st) {
  hipLaunchKernelGGL((pre_bwd_gphi_comp_kernel<N, S, VC, VEC>), dim3((unsigned)ncw, (unsigned)ga.nsplit),
                     dim3(kWave), 0, st, ga);
  return check_launch("pre_bwd_gphi_comp");
}

template <int N, typename S>
static int launch_comp_gphi(const BwdLayout& lay, const PreBwdSmallArgs& sa, float* gphi_part, uint16_t* gpl,
                            float* grad_phi, hipStream_t st) {
  constexpr int VC = N == 4 ? 8 : 4;  // columns per lane: accumulators stay within the VGPR budget
  const int64_t T = sa.T, K = lay.K, ntiles = (T + kCompTile - 1) / kCompTile;
  hipLaunchKernelGGL((comp_gplanes_kernel<N>), dim3(reduce_grid(ntiles * PreDims<N>::MT * kWave)), dim3(256), 0,
                     st, sa.gm, sa.inv_rms, gpl, T, ntiles);
  int rc = check_launch("pre_bwd_comp_gplanes");
  if (rc) return rc;
  // token splits: about 2048 waves, within the partial region (2 floats per
  // output and split)
  const int64_t ncw = (K + 16 * VC - 1) / (16 * VC);
  int64_t ns = (2048 + ncw - 1) / ncw;
  const int64_t cap = dma_max_splits(sa.D) / 2;
  if (ns > cap) ns = cap;
  if (ns > ntiles) ns = ntiles;
  if (ns < 1) ns = 1;
  const int64_t tps = (ntiles + ns - 1) / ns * kCompTile;
  ns = (T + tps - 1) / tps;
  GphiCompArgs ga{sa.x, gpl, gphi_part, T, K, tps, (int)ns};
  const bool vec = K % VC == 0 && aligned16(sa.x) && (K * (int64_t)sizeof(S)) % 16 == 0;
  rc = vec ? launch_comp_gphi_v<N, S, VC, true>(lay, ga, ncw, st) : launch_comp_gphi_v<N, S, VC, false>(lay, ga, ncw, st);
  if (rc) return rc;
  const int64_t n = (int64_t)lay.M * K;
  hipLaunchKernelGGL(sum_splits_comp_kernel, dim3(reduce_grid(n)), dim3(256), 0, st, gphi_part, grad_phi, n,
                     (int)ns);
  return check_launch("pre_bwd_sum_splits_comp");
}

// grad_phi from the split partials (plain) or the compensated kernels, then
// grad_alpha / grad_base
template <int N, typename S>
static int reduce_tail(const BwdLayout& lay, const PreBwdSmallArgs& sa, float* gphi_part, int nsplit,
                       uint16_t* gpl, float* grad_phi, float* grad_alpha, float* grad_base, hipStream_t st) {
  int rc;
  if (sa.comp) {
    rc = launch_comp_gphi<N, S>(lay, sa, gphi_part, gpl, grad_phi, st);
  } else {
    const int64_t n = (int64_t)lay.M * lay.K;
    hipLaunchKernelGGL(sum_splits_kernel, dim3(reduce_grid(n)), dim3(256), 0, st, gphi_part, grad_phi, n,
                       nsplit);
    rc = check_launch("pre_bwd_sum_splits");
  }
  if (rc) return rc;
  return sum_alpha_base(lay, sa, grad_alpha, grad_base, st);
}

// Buffer ranges are 32-bit: one tile of x rows (16 * N * D bf16) must fit.
template <int N>
static bool dma_usable(int D) {
  return (N == 4 || N == 8) && (int64_t)DmaCfg<N>::TT * N * D * 2 < ((int64_t)1 << 31);
}

// Launches the LDS-pipelined kernel; *nsplit receives its token-split count.
template <int N, int P>
static int launch_dma(const BwdLayout& lay, const PreBwdStreamArgs& sta, int* nsplit, hipStream_t st) {
  constexpr int DW = DmaCfg<N>::DW, NG = DmaCfg<N>::NG;
  const int D = sta.D;
  const int64_t ncb = (D + DW - 1) / DW;
  // one block per CU (the ring fills the LDS); as many token splits as fit
  // next to the (column block, stream group) blocks in one wave of blocks
  int64_t ns = device_cu_count() / (ncb * NG);
  if (ns > dma_max_splits(D)) ns = dma_max_splits(D);
  if (ns > lay.ntiles) ns = lay.ntiles;
  if (ns < 1) ns = 1;
  PreBwdDmaArgs da{};
  da.x = sta.x;
  da.gy = sta.gy;
  da.phiT = sta.phiT;
  da.phiT_plane_stride = sta.phiT_plane_stride;
  da.gmP = sta.gmP;
  da.gmP_plane = sta.gmP_plane;
  da.gTw = sta.gTw;
  da.coef = sta.coef;
  da.gx = sta.gx;
  da.gin = sta.gin;
  da.part = sta.gphi_part;
  da.T = sta.T;
  da.D = D;
  da.ntiles = lay.ntiles;
  const dim3 grid((unsigned)(ncb * NG), (unsigned)ns), block(64 * DmaCfg<N>::G);
  // two waves per stream (column halves) at N = 8 (the results are the same
  // bits as with one)
  if (sta.gin)
    hipLaunchKernelGGL((pre_bwd_dma_kernel<N, P, kDmaAccStages, true>), grid, block, 0, st, da);
  else if constexpr (N == 8 && P == 1)
    hipLaunchKernelGGL((pre_bwd_dma_kernel<N, 1, DmaCfg<N>::STAGES, false, 2>), grid, dim3(2 * block.x), 0, st,
                       da);
  else
    hipLaunchKernelGGL((pre_bwd_dma_kernel<N, P, DmaCfg<N>::STAGES, false>), grid, block, 0, st, da);
  *nsplit = (int)ns;
  return check_launch("pre_bwd_dma");
}

// grad_x += grad_x_in for the kernels without an accumulating form
template <typename S>
__global__ void add_into_kernel(S* out, const S* in, int64_t n) {
  for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    store_elem(out, i, load_elem(out, i) + load_elem(in, i));
}

template <typename S>
static int add_into(void* out, const void* in, int64_t n, hipStream_t st) {
  hipLaunchKernelGGL((add_into_kernel<S>), dim3(reduce_grid(n)), dim3(256), 0, st, static_cast<S*>(out),
                     static_cast<const S*>(in), n);
  return check_launch("pre_bwd_add_into");
}

// The single-pass form (pre_bwd_coop.hpp) where it applies: kernel A's SP
// form, the single-pass kernel, then grad_phi and grad_alpha / grad_base in
// fixed order.  *used says whether it ran.
static int launch_pre_bwd_coop(const BwdLayout& lay, PreBwdSmallArgs sa, const PreBwdStreamArgs& sta,
                               float* grad_phi, float* grad_alpha, float* grad_base, char* ws,
                               int32_t* status_out, hipStream_t st, bool* used) {
  *used = false;
  if (!lay.bcG || stream_capturing(st)) return MHC_OK;
  if (!coop_fits((const void*)pre_bwd_coop_kernel, kBcThreads, 1)) return MHC_OK;
  const int grid = device_cu_count();
  if ((int64_t)lay.bcMaxg * lay.bcG > lay.bc_rows) return MHC_OK;  // a contribution row per member
  uint32_t* ctl = reinterpret_cast<uint32_t*>(ws + lay.off_bc_ctl);
  u32x4* ring = reinterpret_cast<u32x4*>(ws + lay.off_bc_ctl + align256((size_t)kCoCtlWords * 4));
  const int64_t words = (int64_t)((align256((size_t)kCoCtlWords * 4) + lay.bc_ring_bytes) / 16);
  hipLaunchKernelGGL(co_zero_kernel, dim3(256), dim3(256), 0, st, reinterpret_cast<u32x4*>(ctl), words);
  int rc = check_launch("pre_bwd_coop_zero");
  if (rc) return rc;
  // the members' contribution rows (group * G + member; rows of groups that
  // do not form stay zero)
  hipLaunchKernelGGL(zero_kernel, dim3(32), dim3(256), 0, st, sa.partial + lay.nblkA * lay.C, lay.bc_rows * lay.C);
  if ((rc = check_launch("pre_bwd_coop_zero_rows"))) return rc;
  // kernel A without the pre head: grad_mixes rows (fp32) and coefX
  sa.gmP = nullptr;
  sa.gTw = nullptr;
  sa.coef = nullptr;
  sa.scale = nullptr;
  sa.gpre_part = nullptr;
  sa.coefX = reinterpret_cast<float*>(ws + lay.off_coef);
  hipLaunchKernelGGL((pre_bwd_small_kernel<4, bf16_t, true, true>), dim3((unsigned)lay.nblkA), dim3(kBwdThreads), 0,
                     st, sa);
  if ((rc = check_launch("pre_bwd_small_sp"))) return rc;
  BwdCoopArgs ca{};
  ca.x = sta.x;
  ca.gy = sta.gy;
  ca.gx = sta.gx;
  ca.phiT = sta.phiT;
  ca.gm = sa.gm;
  ca.coefX = sa.coefX;
  ca.alpha = sa.alpha;
  ca.part = sta.gphi_part;
  ca.contrib = sa.partial + lay.nblkA * lay.C;
  ca.ctl = ctl;
  ca.rec = ring;
  ca.T = sa.T;
  ca.D = sa.D;
  ca.G = lay.bcG;
  ca.maxg = lay.bcMaxg;
  ca.timeout = coop_wait_limit();
  hipLaunchKernelGGL(pre_bwd_coop_kernel, dim3((unsigned)grid), dim3(kBcThreads), 0, st, ca);
  if ((rc = check_launch("pre_bwd_coop"))) return rc;
  *used = true;
  const int64_t n = (int64_t)lay.M * lay.K;
  hipLaunchKernelGGL(bc_sum_kernel, dim3(reduce_grid(n)), dim3(256), 0, st, sta.gphi_part, grad_phi, n, ctl, sta.gx,
                     sa.T * lay.K, status_out);
  if ((rc = check_launch("pre_bwd_coop_sum"))) return rc;
  return sum_alpha_base(lay, sa, grad_alpha, grad_base, st, lay.bc_rows, ctl + kCtlStatus);
}

template <int N, typename S>
static int launch_pre_bwd(const BwdLayout& lay, PreBwdSmallArgs sa, const PreBwdMainArgs& ma,
                          PreBwdStreamArgs sta, float* grad_phi, float* grad_alpha,
                          float* grad_base, bool vec, const void* gin, uint16_t* gpl, hipStream_t st,
                          char* ws, int sp_mode, int32_t* status_out) {
  const dim3 gA((unsigned)lay.nblkA), bA(kBwdThreads);
  const bool streaming = vec && std::is_same<S, bf16_t>::value;
  if constexpr (N == 4 && std::is_same<S, bf16_t>::value) {
    // sp_mode: 0 never, 1 from kBcAutoT tokens, 2 from kBcMinT (the layout's
    // condition)
    const bool single_pass = sp_mode == 2 || (sp_mode == 1 && sa.T >= kBcAutoT);
    if (single_pass && streaming && !gin && !sa.comp && lay.P == 1 && dma_usable<N>(sta.D)) {
      bool used = false;
      const int rc = launch_pre_bwd_coop(lay, sa, sta, grad_phi, grad_alpha, grad_base, ws, status_out, st, &used);
      if (rc || used) return rc;
    }
  }
  if (streaming) {
    if (!sa.comp) sa.gm = nullptr;  // the compensated grad_phi reads fp32 grad_mixes
    sa.scale = nullptr;
  } else {
    sa.gmP = nullptr;
    sa.gTw = nullptr;
    sa.coef = nullptr;
  }
  int rc;
  if (streaming && sa.T >= kGpreDmaMinT) {
    // grad_pre through the LDS-pipelined kernel: one chunk of sums per token
    sa.gpre_part = sa.gpre_buf;
    sa.gpre_chunks = 1;
    hipLaunchKernelGGL((pre_bwd_gpre_dma_kernel<N>), dim3((unsigned)device_cu_count()), dim3(kWave * kGpreDmaWaves),
                       0, st, static_cast<const bf16_t*>(sa.x), static_cast<const bf16_t*>(sa.gy), sa.gpre_buf,
                       sa.T, sa.D);
    if ((rc = check_launch("pre_bwd_gpre_dma"))) return rc;
  } else if (sa.gpre_part) {
    const dim3 gG((unsigned)(sa.T < kGpreGridT ? sa.T : kGpreGridT), (unsigned)lay.gpre_chunks);
    float* part = const_cast<float*>(sa.gpre_part);
    if (vec)
      hipLaunchKernelGGL((pre_bwd_gpre_kernel<N, S, true>), gG, bA, 0, st, sa.x, sa.gy, part, sa.T, sa.D);
    else
      hipLaunchKernelGGL((pre_bwd_gpre_kernel<N, S, false>), gG, bA, 0, st, sa.x, sa.gy, part, sa.T, sa.D);
    if ((rc = check_launch("pre_bwd_gpre"))) return rc;
  }
  if (vec)
    hipLaunchKernelGGL((pre_bwd_small_kernel<N, S, true>), gA, bA, 0, st, sa);
  else
    hipLaunchKernelGGL((pre_bwd_small_kernel<N, S, false>), gA, bA, 0, st, sa);
  rc = check_launch("pre_bwd_small");
  if (rc) return rc;
  if (streaming && dma_usable<N>(sta.D)) {
    sta.gin = static_cast<const bf16_t*>(gin);  // accumulated inside the kernel
    int ns = 0;
    rc = lay.P == 1 ? launch_dma<N, 1>(lay, sta, &ns, st) : launch_dma<N, 2>(lay, sta, &ns, st);
    if (rc) return rc;
    return reduce_tail<N, S>(lay, sa, sta.gphi_part, ns, gpl, grad_phi, grad_alpha, grad_base, st);
  }
  const int64_t nx = sta.T * N * (int64_t)sta.D;
  if (streaming) {
    rc = lay.P == 1 ? launch_stream<N, 1>(lay, sta, st) : launch_stream<N, 2>(lay, sta, st);
    if (rc) return rc;
    if (gin && (rc = add_into<S>(sta.gx, gin, nx, st))) return rc;
    return reduce_tail<N, S>(lay, sa, sta.gphi_part, sta.nsplit, gpl, grad_phi, grad_alpha, grad_base, st);
  }
  const dim3 gB((unsigned)lay.chunks, (unsigned)lay.nsplit), bB(256);
  if (vec)
    hipLaunchKernelGGL((pre_bwd_main_kernel<N, S, true>), gB, bB, 0, st, ma);
  else
    hipLaunchKernelGGL((pre_bwd_main_kernel<N, S, false>), gB, bB, 0, st, ma);
  rc = check_launch("pre_bwd_main");
  if (rc) return rc;
  if (gin && (rc = add_into<S>(ma.gx, gin, nx, st))) return rc;
  return reduce_tail<N, S>(lay, sa, ma.gphi_part, lay.nsplit, gpl, grad_phi, grad_alpha, grad_base, st);
}

template <typename S>
static int dispatch_pre_bwd(int N, const BwdLayout& lay, const PreBwdSmallArgs& sa,
                            const PreBwdMainArgs& ma, const PreBwdStreamArgs& sta, float* gphi,
                            float* galpha, float* gbase, bool vec, const void* gin, uint16_t* gpl,
                            hipStream_t st, char* ws, int sp_mode, int32_t* status_out) {
  switch (N) {
    case 4:
      return launch_pre_bwd<4, S>(lay, sa, ma, sta, gphi, galpha, gbase, vec, gin, gpl, st, ws, sp_mode,
                                  status_out);
    case 8:
      return launch_pre_bwd<8, S>(lay, sa, ma, sta, gphi, galpha, gbase, vec, gin, gpl, st, ws, sp_mode,
                                  status_out);
  }
  return set_error(MHC_ERR_UNSUPPORTED, "mhc_pre_bwd: N=%d not supported (4, 8)", N);
}

}  // namespace mhc

using namespace mhc;

extern "C" size_t mhc_pre_bwd_workspace_size(int64_t T, int32_t N, int32_t D, int32_t phi_dtype,
                                             int32_t iter_times) {
  if (T < 0 || N <= 0 || D <= 0) return 0;
  return bwd_layout(T, N, D, phi_dtype, iter_times).total;
}

static int pre_bwd_entry(const void* x, int32_t x_dtype, const void* phi, int32_t phi_dtype,
                         const float* alpha, const float* base, const float* inv_rms, const float* mixes,
                         const float* pre, const void* grad_y, const float* grad_post_out,
                         const float* grad_comb_frag, float hc_eps, float clamp_min, float clamp_max,
                         int32_t iter_times, const void* grad_x_in, void* grad_x, float* grad_phi,
                         float* grad_alpha, float* grad_base, void* workspace, size_t workspace_bytes,
                         int64_t T, int32_t N, int32_t D, uint32_t flags, int32_t* status, void* stream) {
  clear_error();
  if (flags & ~(uint32_t)(MHC_PRE_BWD_COMPENSATED | MHC_PRE_BWD_TWO_PASS | MHC_PRE_BWD_SINGLE_PASS))
    return set_error(MHC_ERR_INVALID, "mhc_pre_bwd: unknown flags 0x%x", (unsigned)flags);
  if ((flags & MHC_PRE_BWD_TWO_PASS) && (flags & MHC_PRE_BWD_SINGLE_PASS))
    return set_error(MHC_ERR_INVALID, "mhc_pre_bwd: MHC_PRE_BWD_TWO_PASS and MHC_PRE_BWD_SINGLE_PASS together");
  if (T < 0 || D <= 0 || N <= 0)
    return set_error(MHC_ERR_INVALID, "mhc_pre_bwd: bad shape T=%lld N=%d D=%d", (long long)T, N, D);
  if (int rc = check_tokens(T, "mhc_pre_bwd")) return rc;
  if (N != 4 && N != 8) return set_error(MHC_ERR_UNSUPPORTED, "mhc_pre_bwd: N=%d not supported (4, 8)", N);
  if (!phi || !alpha || !base || !grad_phi || !grad_alpha || !grad_base)
    return set_error(MHC_ERR_INVALID, "mhc_pre_bwd: null pointer");
  hipStream_t st = (hipStream_t)stream;
  const int M = 2 * N + N * N;
  if (T == 0) {
    // empty batch: the T-reductions are zero
    hipLaunchKernelGGL(zero_kernel, dim3(64), dim3(256), 0, st, grad_phi, (int64_t)M * N * D);
    hipLaunchKernelGGL(zero_kernel, dim3(1), dim3(64), 0, st, grad_alpha, (int64_t)3);
    hipLaunchKernelGGL(zero_kernel, dim3(1), dim3(64), 0, st, grad_base, (int64_t)M);
    return check_launch("pre_bwd_zero");
  }
  if (!x || !inv_rms || !mixes || !pre || !grad_y || !grad_post_out || !grad_comb_frag || !grad_x)
    return set_error(MHC_ERR_INVALID, "mhc_pre_bwd: null pointer");
  const BwdLayout lay = bwd_layout(T, N, D, phi_dtype, iter_times);
  if (!workspace || workspace_bytes < lay.total)
    return set_error(MHC_ERR_INVALID, "mhc_pre_bwd: workspace too small (%zu < %zu bytes)",
                     workspace_bytes, lay.total);
  char* ws = static_cast<char*>(workspace);
  uint16_t* phiT = reinterpret_cast<uint16_t*>(ws + lay.off_phiT);
  int rc = prepare_phiT_planes(phi, phi_dtype, M, lay.K, phiT, st);
  if (rc) return rc;

  PreBwdSmallArgs sa{};
  sa.x = x;
  sa.gy = grad_y;
  sa.mixes = mixes;
  sa.inv_rms = inv_rms;
  sa.alpha = alpha;
  sa.base = base;
  sa.gpost = grad_post_out;
  sa.gcomb = grad_comb_frag;
  sa.hc_eps = hc_eps;
  sa.cmin = clamp_min;
  sa.cmax = clamp_max;
  sa.apply_clamp = (clamp_min != 0.0f || clamp_max != 0.0f) ? 1 : 0;
  sa.iters = iter_times;
  sa.pre = pre;
  sa.gm = reinterpret_cast<float*>(ws + lay.off_gm);
  sa.scale = reinterpret_cast<float*>(ws + lay.off_scale);
  sa.gmP = reinterpret_cast<uint16_t*>(ws + lay.off_gmP);
  sa.gmP_plane = T * lay.MP32;
  sa.gTw = reinterpret_cast<uint16_t*>(ws + lay.off_gTw);
  sa.coef = reinterpret_cast<float4*>(ws + lay.off_coef);
  sa.partial = reinterpret_cast<float*>(ws + lay.off_partial);
  sa.sink_scratch = reinterpret_cast<float*>(ws + lay.off_sink);
  sa.sink_stride = lay.nblkA * kBwdTile * lay.L;
  sa.gpre_part = lay.gpre_chunks ? reinterpret_cast<float*>(ws + lay.off_gpre) : nullptr;
  sa.gpre_chunks = lay.gpre_chunks;
  sa.gpre_buf = reinterpret_cast<float*>(ws + lay.off_gpre);
  sa.comp = (flags & MHC_PRE_BWD_COMPENSATED) ? 1 : 0;
  sa.T = T;
  sa.D = D;

  PreBwdMainArgs ma{};
  ma.x = x;
  ma.gy = grad_y;
  ma.phiT = phiT;
  ma.phiT_plane_stride = lay.K * lay.MP32;
  ma.phi_planes = lay.P;
  ma.gm = sa.gm;
  ma.inv_rms = inv_rms;
  ma.pre = pre;
  ma.scale = sa.scale;
  ma.gx = grad_x;
  ma.gphi_part = reinterpret_cast<float*>(ws + lay.off_gphi);
  ma.T = T;
  ma.D = D;
  ma.tok_per_split = lay.tok_per_split;

  PreBwdStreamArgs sta{};
  sta.x = static_cast<const bf16_t*>(x);
  sta.gy = static_cast<const bf16_t*>(grad_y);
  sta.phiT = phiT;
  sta.phiT_plane_stride = lay.K * lay.MP32;
  sta.phi_planes = lay.P;
  sta.gmP = sa.gmP;
  sta.gmP_plane = sa.gmP_plane;
  sta.gTw = sa.gTw;
  sta.coef = sa.coef;
  sta.gx = static_cast<bf16_t*>(grad_x);
  sta.gphi_part = ma.gphi_part;
  sta.T = T;
  sta.D = D;

  const bool vec = (D % 8 == 0) && aligned16(x) && aligned16(grad_y) && aligned16(grad_x) &&
                   (!grad_x_in || aligned16(grad_x_in));
  uint16_t* gpl = reinterpret_cast<uint16_t*>(ws + lay.off_gpl);
  const int sp = (flags & MHC_PRE_BWD_TWO_PASS) ? 0 : (flags & MHC_PRE_BWD_SINGLE_PASS) ? 2 : 1;
  switch (x_dtype) {
    case MHC_DTYPE_BF16:
      return dispatch_pre_bwd<bf16_t>(N, lay, sa, ma, sta, grad_phi, grad_alpha, grad_base, vec, grad_x_in, gpl, st,
                                      ws, sp, status);
    case MHC_DTYPE_F16:
      return dispatch_pre_bwd<f16_t>(N, lay, sa, ma, sta, grad_phi, grad_alpha, grad_base, vec, grad_x_in, gpl, st,
                                     ws, sp, status);
    case MHC_DTYPE_F32:
      return dispatch_pre_bwd<float>(N, lay, sa, ma, sta, grad_phi, grad_alpha, grad_base, vec, grad_x_in, gpl, st,
                                     ws, sp, status);
  }
  return set_error(MHC_ERR_UNSUPPORTED, "mhc_pre_bwd: x dtype %d not supported", x_dtype);
}

extern "C" int mhc_pre_bwd(const void* x, int32_t x_dtype, const void* phi, int32_t phi_dtype,
                           const float* alpha, const float* base, const float* inv_rms,
                           const float* mixes, const float* pre, const void* grad_y,
                           const float* grad_post_out, const float* grad_comb_frag, float hc_eps,
                           float clamp_min, float clamp_max, int32_t iter_times, void* grad_x,
                           float* grad_phi, float* grad_alpha, float* grad_base, void* workspace,
                           size_t workspace_bytes, int64_t T, int32_t N, int32_t D,
                           void* stream) {
  return pre_bwd_entry(x, x_dtype, phi, phi_dtype, alpha, base, inv_rms, mixes, pre, grad_y, grad_post_out,
                       grad_comb_frag, hc_eps, clamp_min, clamp_max, iter_times, nullptr, grad_x, grad_phi,
                       grad_alpha, grad_base, workspace, workspace_bytes, T, N, D, 0u, nullptr, stream);
}

// grad_x_in (nullable) must not overlap grad_x
static int check_gin(const void* grad_x_in, const void* grad_x, int64_t T, int32_t N, int32_t D, int32_t x_dtype,
                     const char* who) {
  if (T <= 0 || !grad_x_in || !grad_x) return MHC_OK;
  const uintptr_t bytes = (uintptr_t)T * (uintptr_t)N * (uintptr_t)D * (x_dtype == MHC_DTYPE_F32 ? 4u : 2u);
  const uintptr_t in = (uintptr_t)grad_x_in, out = (uintptr_t)grad_x;
  if (in < out + bytes && out < in + bytes) return set_error(MHC_ERR_INVALID, "%s: grad_x_in overlaps grad_x", who);
  return MHC_OK;
}

extern "C" int mhc_pre_bwd_acc(const void* x, int32_t x_dtype, const void* phi, int32_t phi_dtype,
                               const float* alpha, const float* base, const float* inv_rms,
                               const float* mixes, const float* pre, const void* grad_y,
                               const float* grad_post_out, const float* grad_comb_frag, float hc_eps,
                               float clamp_min, float clamp_max, int32_t iter_times, const void* grad_x_in,
                               void* grad_x, float* grad_phi, float* grad_alpha, float* grad_base,
                               void* workspace, size_t workspace_bytes, int64_t T, int32_t N, int32_t D,
                               void* stream) {
  clear_error();
  if (T > 0 && !grad_x_in) return set_error(MHC_ERR_INVALID, "mhc_pre_bwd_acc: null grad_x_in");
  if (int rc = check_gin(grad_x_in, grad_x, T, N, D, x_dtype, "mhc_pre_bwd_acc")) return rc;
  return pre_bwd_entry(x, x_dtype, phi, phi_dtype, alpha, base, inv_rms, mixes, pre, grad_y, grad_post_out,
                       grad_comb_frag, hc_eps, clamp_min, clamp_max, iter_times, grad_x_in, grad_x, grad_phi,
                       grad_alpha, grad_base, workspace, workspace_bytes, T, N, D, 0u, nullptr, stream);
}

extern "C" int mhc_pre_bwd_ex(const void* x, int32_t x_dtype, const void* phi, int32_t phi_dtype,
                              const float* alpha, const float* base, const float* inv_rms, const float* mixes,
                              const float* pre, const void* grad_y, const float* grad_post_out,
                              const float* grad_comb_frag, float hc_eps, float clamp_min, float clamp_max,
                              int32_t iter_times, const void* grad_x_in, void* grad_x, float* grad_phi,
                              float* grad_alpha, float* grad_base, uint32_t flags, int32_t* status,
                              void* workspace, size_t workspace_bytes, int64_t T, int32_t N, int32_t D,
                              void* stream) {
  clear_error();
  if (int rc = check_gin(grad_x_in, grad_x, T, N, D, x_dtype, "mhc_pre_bwd_ex")) return rc;
  return pre_bwd_entry(x, x_dtype, phi, phi_dtype, alpha, base, inv_rms, mixes, pre, grad_y, grad_post_out,
                       grad_comb_frag, hc_eps, clamp_min, clamp_max, iter_times, grad_x_in, grad_x, grad_phi,
                       grad_alpha, grad_base, workspace, workspace_bytes, T, N, D, flags, status, stream);
}
