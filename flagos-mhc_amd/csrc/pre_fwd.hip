// mhc_pre_clamp_sinkhorn forward, one kernel per call.
//
// Semantics: mhc_pre_clamp_sinkhorn_ref, src/mhc_pre_clamp_sinkhorn.py:974-1022.
//
// A block (4 waves) owns a tile of 16 tokens:
//   1. contraction  acc[t,m] = sum_k x[t,k] * phi[m,k]  (k = n*D + d) on bf16
//      MFMA 16x16x32 (A = 16 tokens x 32 k of x, B = 32 k x 16 m of phi^T),
//      the four waves splitting k; the same pass accumulates sum(x^2).
//      Each lane reads 32 consecutive k of its token row (four 16-byte loads),
//      and the four MFMAs of a step consume those groups in the same order
//      for A and B, so the reduction over k is unaffected by the grouping.
//      mixes = inv_rms * acc, the identity used by the reference's
//      need_backward=False path (src/mhc_pre_clamp_sinkhorn.py:914-916).
//   2. per-token heads and Sinkhorn, one lane per N x N element (sinkhorn.hpp).
//   3. y[t,:] = sum_n pre[t,n] * x[t,n,:], re-reading the tile's x (recently
//      fetched, so mostly served by L2 / the MALL), and optionally the fp32
//      x_scaled = x * inv_rms of the reference's need_backward dict.
// fp16 / fp32 activations and fp16 / fp32 phi are split into two bf16 planes
// each; the products hi*hi + hi*lo + lo*hi keep the contraction within 2^-16
// relative of fp32.
#include "mhc_launch.hpp"
#include "pre_common.hpp"
#include "pre_host.hpp"
#include "sinkhorn.hpp"

namespace mhc {

constexpr int kPreTile = 16;
constexpr int kPreThreads = 256;

struct PreFwdArgs {
  const void* x;
  const uint16_t* phi;       // bf16 planes [P][M][ld]
  int64_t phi_ld;            // row length of a plane (>= K, multiple of 8)
  int64_t phi_plane_stride;  // elements between planes
  int phi_planes;            // 1 or 2
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

template <int N, typename S, bool VEC>
__global__ __launch_bounds__(kPreThreads) void pre_fwd_kernel(PreFwdArgs a) {
  using PD = PreDims<N>;
  constexpr int M = PD::M, MT = PD::MT, MP = PD::MP;
  constexpr int XP = XGroup<S>::PLANES;
  constexpr int L = N * N;

  __shared__ floatx4 red[4][MT][kWave];
  __shared__ float ssq_sh[4][kPreTile];
  __shared__ float mix_sh[kPreTile][MP + 1];
  __shared__ float pre_sh[kPreTile][N];
  __shared__ float inv_sh[kPreTile];

  const S* __restrict__ x = static_cast<const S*>(a.x);
  const int D = a.D;
  const int64_t K = (int64_t)N * D;
  const int tid = threadIdx.x, lane = tid & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, kq = lane >> 4;
  const int64_t t0 = (int64_t)blockIdx.x * kPreTile;
  const bool row_ok = (t0 + r) < a.T;
  const S* xrow = x + (row_ok ? (t0 + r) * K : 0);

  // ---- 1. contraction + sum of squares ----------------------------------
  floatx4 acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) acc[mt] = floatx4{0.f, 0.f, 0.f, 0.f};
  float ssq = 0.f;
  const int P = a.phi_planes;

  for (int64_t kb = (int64_t)wave * 128; kb < K; kb += 4 * 128) {
    const int64_t k = kb + kq * 32;
    u32x4 xp[4][XP];
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      float f[8];
      XGroup<S>::template load<VEC>(xrow, k + 8 * g, K, row_ok, xp[g], f);
#pragma unroll
      for (int i = 0; i < 8; ++i) ssq = fmaf(f[i], f[i], ssq);
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = mt * 16 + r;
      const bool m_ok = m < M;
      for (int p = 0; p < P; ++p) {
        const uint16_t* prow = a.phi + p * a.phi_plane_stride + (m_ok ? m : 0) * a.phi_ld;
        u32x4 b[4];
#pragma unroll
        for (int g = 0; g < 4; ++g)
          b[g] = (m_ok && k + 8 * g < a.phi_ld) ? ld16(prow + k + 8 * g) : zero4();
#pragma unroll
        for (int xi = 0; xi < XP; ++xi) {
          if (xi + p > 1) continue;
#pragma unroll
          for (int g = 0; g < 4; ++g) acc[mt] = mfma16x16x32(as_bf16x8(xp[g][xi]), as_bf16x8(b[g]), acc[mt]);
        }
      }
    }
  }

  ssq += __shfl_xor(ssq, 16, kWave);
  ssq += __shfl_xor(ssq, 32, kWave);
  if (lane < kPreTile) ssq_sh[wave][lane] = ssq;
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) red[wave][mt][lane] = acc[mt];
  __syncthreads();

  // acc layout: lane l holds D[i = 4*(l/16) + v][j = l%16]; i = token, j = m % 16
  for (int idx = tid; idx < kPreTile * MP; idx += kPreThreads) {
    const int tt = idx / MP, m = idx - (idx / MP) * MP;
    const int mt = m >> 4, ln = (m & 15) + 16 * (tt >> 2), v = tt & 3;
    const float s = red[0][mt][ln][v] + red[1][mt][ln][v] + red[2][mt][ln][v] + red[3][mt][ln][v];
    const float ss = ssq_sh[0][tt] + ssq_sh[1][tt] + ssq_sh[2][tt] + ssq_sh[3][tt];
    const float inv = 1.0f / sqrtf(ss / (float)K + a.norm_eps);
    mix_sh[tt][m] = s * inv;
    if (m == 0) inv_sh[tt] = inv;
  }
  __syncthreads();

  if (a.mixes) {
    for (int idx = tid; idx < kPreTile * M; idx += kPreThreads) {
      const int tt = idx / M, m = idx - (idx / M) * M;
      if (t0 + tt < a.T) a.mixes[(t0 + tt) * M + m] = mix_sh[tt][m];
    }
  }
  if (a.inv_rms && tid < kPreTile && t0 + tid < a.T) a.inv_rms[t0 + tid] = inv_sh[tid];

  // ---- 2. heads + Sinkhorn, lane per matrix element -----------------------
  {
    constexpr int TPP = kPreThreads / L;  // tokens per pass
    constexpr int PASSES = kPreTile / TPP;
    const float a0 = a.alpha[0], a1 = a.alpha[1], a2 = a.alpha[2];
#pragma unroll
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
  S* __restrict__ y = static_cast<S*>(a.y);
  const int DG = (D + 7) / 8;
  for (int u = tid; u < kPreTile * DG; u += kPreThreads) {
    const int tt = u / DG, dg = u - (u / DG) * DG;
    const int64_t tok = t0 + tt;
    if (tok >= a.T) break;
    const int64_t d = (int64_t)dg * 8;
    float o[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = 0.f;
    const float inv = inv_sh[tt];
#pragma unroll
    for (int n = 0; n < N; ++n) {
      float f[8];
      load8f<S, VEC>(x + (tok * N + n) * D, d, D, true, f);
      const float p = pre_sh[tt][n];
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = fmaf(p, f[i], o[i]);
      if (a.x_scaled) {
        float xs[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) xs[i] = f[i] * inv;
        store8<float, VEC>(a.x_scaled + tok * K + (int64_t)n * D, d, D, xs);
      }
    }
    store8<S, VEC>(y + tok * D, d, D, o);
  }
}

template <int N, typename S>
static int launch_pre_fwd(const PreFwdArgs& a, bool vec, hipStream_t st) {
  const dim3 grid((unsigned)((a.T + kPreTile - 1) / kPreTile)), block(kPreThreads);
  if (vec)
    hipLaunchKernelGGL((pre_fwd_kernel<N, S, true>), grid, block, 0, st, a);
  else
    hipLaunchKernelGGL((pre_fwd_kernel<N, S, false>), grid, block, 0, st, a);
  return check_launch("pre_fwd");
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
