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

extern "C" size_t mhc_pre_fwd_workspace_size(int64_t T, int32_t N, int32_t D, int32_t phi_dtype) {
  (void)T;
  if (N <= 0 || D <= 0) return 0;
  const int M = 2 * N + N * N;
  const int64_t K = (int64_t)N * D;
  if (phi_dtype == MHC_DTYPE_BF16 && K % 8 == 0) return 256;  // used directly when aligned
  return align256(phi_planes_bytes(phi_dtype, M, K));
}

extern "C" int mhc_pre_fwd(const void* x, int32_t x_dtype, const void* phi, int32_t phi_dtype,
                           const float* alpha, const float* base, float norm_eps, float hc_eps,
                           float clamp_min, float clamp_max, int32_t iter_times, void* y,
                           float* post_out, float* comb_frag, float* inv_rms, float* mixes,
                           float* h_res_logits, float* pre, float* x_scaled, void* workspace,
                           size_t workspace_bytes, int64_t T, int32_t N, int32_t D,
                           void* stream) {
  clear_error();
  if (T < 0 || D <= 0 || N <= 0)
    return set_error(MHC_ERR_INVALID, "mhc_pre_fwd: bad shape T=%lld N=%d D=%d", (long long)T, N, D);
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
  const bool vec = (D % 8 == 0) && aligned16(x) && aligned16(y) && (!x_scaled || aligned16(x_scaled));
  switch (x_dtype) {
    case MHC_DTYPE_BF16: return dispatch_pre_fwd<bf16_t>(N, a, vec, st);
    case MHC_DTYPE_F16: return dispatch_pre_fwd<f16_t>(N, a, vec, st);
    case MHC_DTYPE_F32: return dispatch_pre_fwd<float>(N, a, vec, st);
  }
  return set_error(MHC_ERR_UNSUPPORTED, "mhc_pre_fwd: x dtype %d not supported", x_dtype);
}
