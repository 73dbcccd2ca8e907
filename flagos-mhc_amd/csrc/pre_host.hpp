// Host-side helpers of the pre-op entry points: workspace layout and the
// preparation of phi as bf16 MFMA operand planes.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace mhc {

inline size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }
inline int64_t round_up(int64_t v, int64_t m) { return (v + m - 1) / m * m; }

// bf16 planes carrying phi in the forward contraction: 1 for bf16, 2 for fp16
// (exact), 3 for fp32 (residual below 2^-26, so mixes keep fp32 accuracy).
inline int phi_fwd_planes(int32_t phi_dtype) {
  return phi_dtype == 1 /*BF16*/ ? 1 : (phi_dtype == 2 /*F16*/ ? 2 : 3);
}
// Planes of phi^T in the backward (grad_mixes @ phi feeds the x-dtype grad_x):
// 1 for bf16, 2 otherwise.
inline int phi_bwd_planes(int32_t phi_dtype) { return phi_dtype == 1 ? 1 : 2; }

// Bytes of phi planes laid out [P][M][round_up(K, 8)].
inline size_t phi_planes_bytes(int32_t phi_dtype, int M, int64_t K) {
  return (size_t)phi_fwd_planes(phi_dtype) * (size_t)M * (size_t)round_up(K, 8) * 2;
}

// Bytes of transposed phi planes laid out [P][K][MP32], MP32 = M rounded up to 32.
inline size_t phiT_planes_bytes(int32_t phi_dtype, int M, int64_t K) {
  return (size_t)phi_bwd_planes(phi_dtype) * (size_t)K * (size_t)round_up(M, 32) * 2;
}

// y = sum_n pre[t, n] * x[t, n, :] for bf16 x (T, N, D), D % 8 == 0 and
// 16-byte aligned rows (the pre forward's y kernel, a block per token); pre
// (T, N) fp32 in device memory.  The fused post + pre forward runs it on
// x_next.
int launch_pre_y_pass(const void* x, const float* pre, void* y, int64_t T, int N, int D, hipStream_t st);

// Whether mhc_pre_fwd without x_scaled runs its single-pass form (x read
// from HBM once) on these arguments: N = 4, bf16 x and phi, a slice
// geometry for D, T large enough, workspace for it, no stream capture.
bool pre_fwd_single_pass_applies(const void* x, int32_t x_dtype, const void* phi, int32_t phi_dtype, const void* y,
                                 size_t workspace_bytes, int64_t T, int32_t N, int32_t D, hipStream_t st);

// The fused post + pre forward in one pass (N = 4, bf16): x_next formed in
// the single-pass pre kernel and written once.  *used is false (and nothing
// ran) where that form does not apply.  `status` (may be null) receives the
// single pass's status word, as mhc_pre_fwd_ex's.
int post_pre_fwd_single_pass(const void* x, const float* h_res, const void* h_out, const float* h_post,
                             const void* phi, const float* alpha, const float* base, float norm_eps, float hc_eps,
                             float clamp_min, float clamp_max, int32_t iter_times, void* x_next, void* y,
                             float* post_out, float* comb_frag, float* inv_rms, float* mixes, float* h_res_logits,
                             float* pre, void* workspace, size_t workspace_bytes, int32_t* status, int64_t T,
                             int32_t D, hipStream_t st, bool* used);

// Bytes the pre forward (and the fused post + pre forward) keep per call for
// pre (T, N) and inv_rms (T,) between their contraction and y kernels.
inline size_t fwd_y_ws_bytes(int64_t T, int N) { return align256((size_t)T * N * 4) + align256((size_t)T * 4); }

// Makes phi available as bf16 planes [P][M][ld].  bf16 phi with K % 8 == 0
// and a 16-byte aligned base is used in place; anything else is converted
// into `ws` (which must hold phi_planes_bytes).
int prepare_phi_planes(const void* phi, int32_t phi_dtype, int M, int64_t K, void* ws,
                       size_t ws_bytes, const uint16_t** planes, int64_t* ld,
                       int64_t* plane_stride, int* nplanes, hipStream_t st);

// Writes phi^T as bf16 planes [P][K][MP32] (zero for m >= M) into `dst`.
int prepare_phiT_planes(const void* phi, int32_t phi_dtype, int M, int64_t K, uint16_t* dst,
                        hipStream_t st);

}  // namespace mhc
