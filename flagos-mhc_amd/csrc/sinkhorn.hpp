// Per-token N x N Sinkhorn stage, one lane per matrix element.
//
// A token's matrix occupies N*N consecutive lanes of a wave64 (lane offset a
// multiple of N*N), element (i, j) on lane base + i*N + j.  Row sums reduce
// over the j bits of the lane index, column sums over the i bits, both with
// xor shuffles, so the whole stage stays in registers: N=4 packs four tokens
// per wave, N=8 one token per wave.
//
// Forward (src/mhc_pre_clamp_sinkhorn.py:1001-1010):
//   s = softmax_row(lc);  C0 = (s + eps) / (colsum(s + eps) + eps)
//   repeat iters-1:  R = C / (rowsum(C) + eps);  C = R / (colsum(R) + eps)
// Backward: the reference differentiates that loop with torch autograd
// (src/mhc_pre_clamp_sinkhorn_backward.py:1440-1453); here the normalisation
// VJP  du = inv * (g - sum(g * out))  is applied along columns / rows in
// reverse order, using the column-normalised states C_k kept in registers
// (iters <= kSinkRegIters) or in caller scratch (longer runs).  Both
// directions divide by multiplying with v_rcp_f32 (1 ulp) instead of the
// correctly rounded division sequence (about ten instructions each, half of
// the VJP's instructions): states, output and gradient differ from exactly
// rounded ones by a few ulp, far inside the tolerances.
#pragma once

#include "common.hpp"

namespace mhc {

constexpr int kSinkRegIters = 32;

template <int N> struct SinkLanes {
  static constexpr int L = N * N;                       // lanes per token
  static constexpr int ROW = N - 1;                     // xor mask over j bits
  static constexpr int COL = (L - 1) & ~(N - 1);        // xor mask over i bits
  static_assert((N & (N - 1)) == 0 && L <= kWave, "N must be a power of two, N*N <= 64");
};

// 1 / s by v_rcp_f32 (s >= eps > 0 here: no denormal or zero inputs)
__device__ __forceinline__ float rcp1(float s) { return __builtin_amdgcn_rcpf(s); }

// One (row, column) normalisation pair C_{k-1} -> C_k, the softmax output
// (without eps) of this lane's row, and the first column normalisation.
template <int N>
__device__ __forceinline__ float sink_step_r(float c, float eps) {
  const float r = c * rcp1(group_sum<SinkLanes<N>::ROW>(c) + eps);
  return r * rcp1(group_sum<SinkLanes<N>::COL>(r) + eps);
}
template <int N>
__device__ __forceinline__ float sink_softmax_r(float lc) {
  const float mx = group_max<SinkLanes<N>::ROW>(lc);
  const float e = expf(lc - mx);
  return e * rcp1(group_sum<SinkLanes<N>::ROW>(e));
}
template <int N>
__device__ __forceinline__ float sink_first_r(float s, float eps) {
  const float m0 = s + eps;
  return m0 * rcp1(group_sum<SinkLanes<N>::COL>(m0) + eps);
}

// Forward only; returns this lane's comb_frag element.
template <int N>
__device__ float sinkhorn_fwd(float lc, float eps, int iters) {
  float c = sink_first_r<N>(sink_softmax_r<N>(lc), eps);
  for (int k = 1; k < iters; ++k) c = sink_step_r<N>(c, eps);
  return c;
}

// VJP through  out = u / s  with s = sum(u) + eps along the lanes of MASK,
// given out, s and the incoming gradient g.
template <int MASK>
__device__ __forceinline__ float norm_vjp(float g, float out, float s) {
  return rcp1(s) * (g - group_sum<MASK>(g * out));
}

// Backward of one step C_k = colnorm(rownorm(C_{k-1})): given C_{k-1} and
// dL/dC_k, returns dL/dC_{k-1}.
template <int N>
__device__ __forceinline__ float sink_step_vjp(float cprev, float g, float eps) {
  constexpr int ROW = SinkLanes<N>::ROW, COL = SinkLanes<N>::COL;
  // each group sum once: the recomputed forward's denominators serve the VJP
  const float sr = group_sum<ROW>(cprev) + eps;
  const float r = cprev * rcp1(sr);
  const float sc = group_sum<COL>(r) + eps;
  const float c = r * rcp1(sc);
  return norm_vjp<ROW>(norm_vjp<COL>(g, c, sc), r, sr);
}

// Backward of softmax + eps + first column normalisation: given the softmax
// output s and dL/dC_0, returns dL/d(clamped logit).
template <int N>
__device__ __forceinline__ float sink_first_vjp(float s, float g, float eps) {
  constexpr int ROW = SinkLanes<N>::ROW, COL = SinkLanes<N>::COL;
  const float m0 = s + eps;
  const float s0 = group_sum<COL>(m0) + eps;
  const float gm = norm_vjp<COL>(g, m0 * rcp1(s0), s0);
  return s * (gm - group_sum<ROW>(gm * s));
}

// Full VJP of sinkhorn_fwd with respect to the clamped logit of this lane.
// Register path: states C_0 .. C_{iters-2} live in a fully unrolled array.
template <int N>
__device__ float sinkhorn_vjp_regs(float lc, float g, float eps, int iters) {
  float st[kSinkRegIters];
  const float s = sink_softmax_r<N>(lc);
  st[0] = sink_first_r<N>(s, eps);
#pragma unroll
  for (int k = 1; k < kSinkRegIters; ++k)
    if (k < iters - 1) st[k] = sink_step_r<N>(st[k - 1], eps);
#pragma unroll
  for (int k = kSinkRegIters - 1; k >= 1; --k)
    if (k < iters) g = sink_step_vjp<N>(st[k - 1], g, eps);
  return sink_first_vjp<N>(s, g, eps);
}

// Scratch path for iters > kSinkRegIters: states go to a per-lane strided
// buffer (stride = lanes in flight), written forward and read in reverse.
template <int N>
__device__ float sinkhorn_vjp_scratch(float lc, float g, float eps, int iters, float* buf,
                                      int64_t stride) {
  const float s = sink_softmax_r<N>(lc);
  float c = sink_first_r<N>(s, eps);
  for (int k = 0; k < iters - 1; ++k) {
    buf[k * stride] = c;
    c = sink_step_r<N>(c, eps);
  }
  for (int k = iters - 1; k >= 1; --k) g = sink_step_vjp<N>(buf[(k - 1) * stride], g, eps);
  return sink_first_vjp<N>(s, g, eps);
}

__device__ __forceinline__ float sigmoidf_(float z) { return 1.0f / (1.0f + expf(-z)); }

// inv_rms of a token from its sum of squares over k = N*D values, and the
// pre gate sigma(mix * alpha0 + base) + hc_eps, written once so every kernel
// that forms them (the finalize kernel and the single-pass forward, which
// uses pre for y before the finalize kernel writes it out) rounds alike.
__device__ __forceinline__ float rms_inv(float ssq, float k, float eps) { return 1.0f / sqrtf(ssq / k + eps); }
__device__ __forceinline__ float pre_gate(float mix, float a0, float base, float hc_eps) {
  return sigmoidf_(fmaf(mix, a0, base)) + hc_eps;
}

__device__ __forceinline__ float clamp_logit(float l, int apply, float lo, float hi) {
  // torch.clamp(l, lo, hi) == min(max(l, lo), hi)
  return apply ? fminf(fmaxf(l, lo), hi) : l;
}

}  // namespace mhc
