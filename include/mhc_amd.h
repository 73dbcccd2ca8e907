/*
 * mhc_amd.h -- C ABI of the MI355X (gfx950) mHC operator library
 * (libmhc_amd.so).
 *
 * The reference (liuhycs/FlagOS-mhc) is a Python operator package with no
 * FFI; its boundary is the Python API of src/__init__.py:34-47.  Each entry
 * point below replaces the device work behind one of its four operators, and
 * the Python package FlagOS_mhc binds them with ctypes exactly as a
 * maintainer of the reference would (see FlagOS_mhc/_lib.py).
 *
 * Conventions (all entry points):
 *   - plain device pointers and sizes; the library never allocates or
 *     frees memory: scratch space is passed in by the caller as `workspace`
 *     (size from the matching *_workspace_size call), except for
 *     mhc_pre_fwd_noalloc, whose workspace is a static per-GPU array;
 *   - every tensor is contiguous, row-major, in the (T, N, D) token layout
 *     (T = tokens = B*S, N = streams, D = width); gates and Sinkhorn
 *     quantities are fp32;
 *   - work is enqueued on `stream` (a hipStream_t; NULL = default stream)
 *     and nothing synchronises with the host;
 *   - return MHC_OK (0) or a negative MHC_ERR_* code; mhc_last_error()
 *     then returns a message (thread-local, valid until the next call);
 *   - T == 0 is accepted and does nothing.
 */
#ifndef MHC_AMD_H_
#define MHC_AMD_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* storage dtypes of activations (x, h_out, y, grads) and of phi */
#define MHC_DTYPE_F32 0
#define MHC_DTYPE_BF16 1
#define MHC_DTYPE_F16 2

#define MHC_OK 0
#define MHC_ERR_INVALID (-1)     /* bad argument: shape, null pointer, size */
#define MHC_ERR_UNSUPPORTED (-2) /* valid but not implemented (e.g. N) */
#define MHC_ERR_HIP (-3)         /* HIP runtime error (launch failure) */

/* Message describing the last failure on this thread ("" if none). */
const char* mhc_last_error(void);

/* Library version, major*10000 + minor*100 + patch. */
int32_t mhc_version(void);

/*
 * mhc_post forward.  Replaces the device work of mhc_post
 * (src/mhc_post.py:296-341; semantics of mhc_post_ref, :344-352):
 *   y[t,i,:] = sum_j h_res[t,j,i] * x[t,j,:] + h_post[t,i] * h_out[t,:]
 * x, y: (T,N,D) `dtype`; h_out: (T,D) `dtype`; h_res: (T,N,N) fp32;
 * h_post: (T,N) fp32.  N in {2,4,6,8}.
 */
int mhc_post_fwd(const void* x, const float* h_res, const void* h_out, const float* h_post,
                 void* y, int64_t T, int32_t N, int32_t D, int32_t dtype, void* stream);

/*
 * mhc_post backward.  Replaces the device work of mhc_post_backward
 * (src/mhc_post_backward.py:593-621; semantics of mhc_post_backward_ref,
 * :624-643).  grad_y, x, grad_x: (T,N,D) `dtype`; h_out, grad_h_out: (T,D)
 * `dtype`; h_res, grad_h_res: (T,N,N) fp32; h_post, grad_h_post: (T,N) fp32.
 */
int mhc_post_bwd(const void* grad_y, const void* x, const float* h_res, const void* h_out,
                 const float* h_post, void* grad_x, float* grad_h_res, void* grad_h_out,
                 float* grad_h_post, int64_t T, int32_t N, int32_t D, int32_t dtype,
                 void* stream);

/*
 * mhc_post backward for the incoming gradient grad_y + grad_y2 (both (T,N,D)
 * `dtype`, added in fp32 as they are read; other arguments as mhc_post_bwd).
 * No counterpart in the reference: it serves the backward of a fused
 * post(l) + pre(l+1) layer, where x_next's gradient has two parts (the one
 * that reaches x_next directly and the pre backward's grad_x) and the post
 * backward of layer l reads both instead of a kernel writing their sum.
 */
int mhc_post_bwd_sum(const void* grad_y, const void* grad_y2, const void* x, const float* h_res,
                     const void* h_out, const float* h_post, void* grad_x, float* grad_h_res,
                     void* grad_h_out, float* grad_h_post, int64_t T, int32_t N, int32_t D,
                     int32_t dtype, void* stream);

/*
 * 1 when mhc_post_bwd_sum runs the kernel form mhc_post_bwd runs for this
 * shape (16-byte aligned rows), plus one read; 0 when that form has no
 * summed variant (N = 4 bf16, T >= 1024, D < 2048) and mhc_post_bwd_sum takes
 * a slower one.  No counterpart in the reference.
 */
int mhc_post_bwd_sum_fused(int64_t T, int32_t N, int32_t D, int32_t dtype);

/*
 * mhc_pre_clamp_sinkhorn forward.  Replaces the device work of
 * mhc_pre_clamp_sinkhorn (src/mhc_pre_clamp_sinkhorn.py:857-971; semantics of
 * mhc_pre_clamp_sinkhorn_ref, :974-1022): RMSNorm over N*D, the N*D -> M
 * contraction with phi (M = 2N + N^2), sigmoid heads, optional clamp (on iff
 * clamp_min != 0 or clamp_max != 0), row softmax and iter_times Sinkhorn
 * normalisations, y = sum_n x[n] * pre[n].
 * x: (T,N,D) `x_dtype`; phi: (M, N*D) `phi_dtype`; alpha (3,), base (M,) fp32.
 * Outputs: y (T,D) `x_dtype`; post_out (T,N), comb_frag (T,N,N) fp32.
 * Optional outputs (may be NULL): inv_rms (T,), mixes (T,M), h_res_logits
 * (T,N,N) pre-clamp, pre (T,N), x_scaled (T,N*D) -- all fp32.
 * N in {4, 8}.  Any D >= 1; D % 8 == 0 with 16-byte aligned rows takes the
 * vectorised path.  mhc_pre_fwd_workspace_size includes, for N = 4 with bf16
 * x and phi, D = 4096 or 7168 .. 8192 and T >= 8192, the exchange ring of the
 * single-pass form (x read from HBM once, ~13 MB + 120 bytes per token); a
 * smaller workspace that still holds the two-pass forms' runs those.
 */
size_t mhc_pre_fwd_workspace_size(int64_t T, int32_t N, int32_t D, int32_t phi_dtype);
int mhc_pre_fwd(const void* x, int32_t x_dtype, const void* phi, int32_t phi_dtype,
                const float* alpha, const float* base, float norm_eps, float hc_eps,
                float clamp_min, float clamp_max, int32_t iter_times, void* y, float* post_out,
                float* comb_frag, float* inv_rms, float* mixes, float* h_res_logits, float* pre,
                float* x_scaled, void* workspace, size_t workspace_bytes, int64_t T, int32_t N,
                int32_t D, void* stream);

/*
 * mhc_pre_fwd with a status word.  The single-pass form's waits for the other
 * CUs of its group are bounded (0.25 s without progress); if one gives up
 * (the GPU was preempted or shared for that long), every output of the call
 * is NaN, and the kernels write the failure code (> 0) to *status, or 0 when
 * every wait was satisfied.  Other forms have no such waits and leave *status
 * untouched, so the caller zeroes it first.  `status` may be a device pointer
 * or host-mapped pinned memory (hipHostMalloc); it is written when the call's
 * work runs, so the caller reads it after synchronising with `stream`.
 * mhc_pre_fwd is this call with status == NULL: it returns MHC_OK before the
 * kernels run and cannot report such a failure.  No counterpart in the
 * reference (its Triton kernels have no cross-CU waits; its failures are
 * host exceptions, src/mhc_pre_clamp_sinkhorn.py:884-889).  Other arguments
 * as in mhc_pre_fwd.
 */
int mhc_pre_fwd_ex(const void* x, int32_t x_dtype, const void* phi, int32_t phi_dtype,
                   const float* alpha, const float* base, float norm_eps, float hc_eps,
                   float clamp_min, float clamp_max, int32_t iter_times, void* y, float* post_out,
                   float* comb_frag, float* inv_rms, float* mixes, float* h_res_logits, float* pre,
                   float* x_scaled, void* workspace, size_t workspace_bytes, int32_t* status,
                   int64_t T, int32_t N, int32_t D, void* stream);

/*
 * Test hook, no counterpart in the reference: sets the limit of the
 * single-pass form's bounded waits to `ticks` of the GPU's 100 MHz clock for
 * every later call in this process (0 makes every wait that is not already
 * satisfied give up at once, which forces the failure path above); a
 * negative value restores the default (0.25 s).  Nothing else sets it.
 */
void mhc_debug_set_wait_limit(int64_t ticks);

/*
 * mhc_pre_fwd without a workspace argument.  No counterpart in the reference:
 * it is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  It calls
 * no hipMalloc / hipFree or other allocating routine: the workspace is a
 * static device array of MHC_PRE_FWD_SCRATCH_BYTES per GPU, held until the
 * process ends.  Calls whose two-pass workspace exceeds it are refused with
 * MHC_ERR_INVALID (N = 4, bf16 phi: above about 3.3 M tokens); where the
 * single-pass form's larger workspace fits too (N = 4, bf16, D = 4096 or
 * 7168 .. 8192, T from 8192 to about 450 K tokens) that form runs, as in
 * mhc_pre_fwd with a full workspace.  The
 * current device must be the one `stream` and the tensors belong to.  Every
 * call on a GPU shares that GPU's array: calls that overlap on one GPU (other
 * streams or threads) race.  Arguments and outputs as in mhc_pre_fwd.
 */
#define MHC_PRE_FWD_SCRATCH_BYTES (64u << 20)
int mhc_pre_fwd_noalloc(const void* x, int32_t x_dtype, const void* phi, int32_t phi_dtype,
                        const float* alpha, const float* base, float norm_eps, float hc_eps,
                        float clamp_min, float clamp_max, int32_t iter_times, void* y,
                        float* post_out, float* comb_frag, float* inv_rms, float* mixes,
                        float* h_res_logits, float* pre, float* x_scaled, int64_t T, int32_t N,
                        int32_t D, void* stream);

/*
 * mhc_pre_clamp_sinkhorn backward.  Replaces the device work of
 * mhc_pre_clamp_sinkhorn_backward
 * (src/mhc_pre_clamp_sinkhorn_backward.py:1292-1391; semantics of
 * mhc_pre_clamp_sinkhorn_backward_ref, :1397-1453).  Takes the forward's
 * saved inv_rms (T,), mixes (T,M) and pre (T,N); the reference's x_scaled and
 * h_res_logits are not needed (x * inv_rms and the logits are recomputed).
 * grad_y: (T,D) `x_dtype`; grad_post_out (T,N), grad_comb_frag (T,N,N) fp32.
 * Outputs: grad_x (T,N,D) `x_dtype`; grad_phi (M,N*D), grad_alpha (3,),
 * grad_base (M,) fp32.  The T-reductions are deterministic (fixed order).
 * iter_times above 32 keeps the Sinkhorn states in workspace rather than in
 * registers, which is why the workspace size depends on it.
 */
size_t mhc_pre_bwd_workspace_size(int64_t T, int32_t N, int32_t D, int32_t phi_dtype,
                                  int32_t iter_times);
int mhc_pre_bwd(const void* x, int32_t x_dtype, const void* phi, int32_t phi_dtype,
                const float* alpha, const float* base, const float* inv_rms, const float* mixes,
                const float* pre, const void* grad_y, const float* grad_post_out,
                const float* grad_comb_frag, float hc_eps, float clamp_min, float clamp_max,
                int32_t iter_times, void* grad_x, float* grad_phi, float* grad_alpha,
                float* grad_base, void* workspace, size_t workspace_bytes, int64_t T, int32_t N,
                int32_t D, void* stream);

/*
 * mhc_pre_bwd that accumulates: grad_x = grad_x_in + dL/dx, in one pass for
 * N = 4 bf16 with 16-byte aligned rows (other shapes add in a second kernel).
 * No counterpart in the reference; it is for callers that sum the pre
 * backward's grad_x with another gradient of the same x (the fused post + pre
 * layer below: the residual-stream gradient reaching x_next), which otherwise
 * takes a separate read-read-write pass.  grad_x_in: (T,N,D) `x_dtype`; it
 * must not overlap grad_x.  Other arguments as in mhc_pre_bwd.
 */
int mhc_pre_bwd_acc(const void* x, int32_t x_dtype, const void* phi, int32_t phi_dtype,
                    const float* alpha, const float* base, const float* inv_rms,
                    const float* mixes, const float* pre, const void* grad_y,
                    const float* grad_post_out, const float* grad_comb_frag, float hc_eps,
                    float clamp_min, float clamp_max, int32_t iter_times, const void* grad_x_in,
                    void* grad_x, float* grad_phi, float* grad_alpha, float* grad_base,
                    void* workspace, size_t workspace_bytes, int64_t T, int32_t N, int32_t D,
                    void* stream);

/*
 * mhc_pre_bwd with options.  grad_x_in may be NULL (then as mhc_pre_bwd) or
 * as in mhc_pre_bwd_acc.  flags:
 *   MHC_PRE_BWD_COMPENSATED  compensated T-reductions for grad_phi,
 *       grad_alpha and grad_base: the production AscendC operator's
 *       deterministic Kahan-summation mode, which the reference lists as not
 *       replicated (README.md:197-204, "Deterministic mode and Kahan
 *       compensated summation in mhc_pre_clamp_sinkhorn_backward").  grad_phi
 *       is formed from exact 16-token products (grad_mixes * inv_rms in three
 *       bf16 planes, x in one to three) added with Neumaier's compensation;
 *       grad_alpha / grad_base partials likewise.  Results stay deterministic;
 *       grad_x is unchanged.  Costs one more read of x.
 *   MHC_PRE_BWD_TWO_PASS  never the single-pass form below (for comparisons).
 *   MHC_PRE_BWD_SINGLE_PASS  the single-pass form wherever its conditions
 *       hold (the default choice too).
 * Unknown flag bits, or both pass flags, are an error.  Workspace:
 * mhc_pre_bwd_workspace_size.
 *
 * Single-pass form.  For N = 4 with bf16 x, grad_y and phi, 16-byte aligned
 * rows, D = 4096 or 7168 .. 8192, T >= 8192 (measured faster than the
 * two-pass forms there on MI355X), no grad_x_in, no compensated
 * mode and no stream capture, x and grad_y are read from HBM once (groups of
 * CUs of one XCC share each 16-token tile and exchange per-token grad_pre
 * partials through L2).  Its waits for the other CUs of a group are bounded
 * (0.25 s without progress); if one gives up, grad_x, grad_phi, grad_alpha
 * and grad_base are NaN and the kernels write the failure code (> 0) to
 * *status, else 0.  Other forms leave *status untouched (the caller zeroes
 * it first).  `status` may be NULL, a device pointer or host-mapped pinned
 * memory; it is written when the call's work runs.  mhc_pre_bwd and
 * mhc_pre_bwd_acc run the same forms with status == NULL.
 */
#define MHC_PRE_BWD_COMPENSATED 1u
#define MHC_PRE_BWD_TWO_PASS 2u
#define MHC_PRE_BWD_SINGLE_PASS 4u
int mhc_pre_bwd_ex(const void* x, int32_t x_dtype, const void* phi, int32_t phi_dtype,
                   const float* alpha, const float* base, const float* inv_rms, const float* mixes,
                   const float* pre, const void* grad_y, const float* grad_post_out,
                   const float* grad_comb_frag, float hc_eps, float clamp_min, float clamp_max,
                   int32_t iter_times, const void* grad_x_in, void* grad_x, float* grad_phi,
                   float* grad_alpha, float* grad_base, uint32_t flags, int32_t* status,
                   void* workspace, size_t workspace_bytes, int64_t T, int32_t N, int32_t D,
                   void* stream);

/*
 * Fused forward of mhc_post (layer l) and mhc_pre_clamp_sinkhorn (layer l+1).
 * No single counterpart in the reference: it replaces the device work of
 * mhc_post (src/mhc_post.py:296-352) followed by mhc_pre_clamp_sinkhorn on its
 * output (src/mhc_pre_clamp_sinkhorn.py:857-971), the pair the reference's
 * model code runs between two sublayers.
 * x: (T,N,D), h_out: (T,D) `x_dtype`; h_res (T,N,N), h_post (T,N) fp32;
 * phi, alpha, base, eps / clamp / iter_times as in mhc_pre_fwd.
 * Outputs: x_next = mhc_post(x, h_res, h_out, h_post) (T,N,D) `x_dtype`,
 * bit-identical to mhc_post_fwd; y, post_out, comb_frag and the optional
 * inv_rms, mixes, h_res_logits, pre of mhc_pre_fwd applied to x_next (no
 * x_scaled).  N = 4 with bf16 x, h_out and phi and 16-byte aligned rows:
 * where mhc_pre_fwd has its single pass (T >= 8192, D = 4096 or 7168..8192,
 * the workspace from mhc_post_pre_fwd_workspace_size, no stream capture)
 * that kernel forms x_next itself (x and h_out read once, x_next written
 * once; outputs bit-identical to the two operators); other shapes with
 * D % 64 == 0 and D >= 256 read x once and write x_next once, then read
 * x_next back for y; every other shape runs mhc_post_fwd then mhc_pre_fwd.
 */
size_t mhc_post_pre_fwd_workspace_size(int64_t T, int32_t N, int32_t D, int32_t phi_dtype);
int mhc_post_pre_fwd(const void* x, const float* h_res, const void* h_out, const float* h_post,
                     int32_t x_dtype, const void* phi, int32_t phi_dtype, const float* alpha,
                     const float* base, float norm_eps, float hc_eps, float clamp_min,
                     float clamp_max, int32_t iter_times, void* x_next, void* y, float* post_out,
                     float* comb_frag, float* inv_rms, float* mixes, float* h_res_logits,
                     float* pre, void* workspace, size_t workspace_bytes, int64_t T, int32_t N,
                     int32_t D, void* stream);
/*
 * mhc_post_pre_fwd with a status word, as mhc_pre_fwd_ex: where the single
 * pass runs (the one-pass fused form, or mhc_pre_fwd's single pass after
 * mhc_post_fwd) a bounded wait that gives up makes every output of the call
 * NaN (x_next included) and writes its failure code (> 0) to *status, 0 when
 * every wait was satisfied; other forms leave *status untouched.
 * mhc_post_pre_fwd is this call with status == NULL.  No counterpart in the
 * reference.  Other arguments as in mhc_post_pre_fwd.
 */
int mhc_post_pre_fwd_ex(const void* x, const float* h_res, const void* h_out, const float* h_post,
                        int32_t x_dtype, const void* phi, int32_t phi_dtype, const float* alpha,
                        const float* base, float norm_eps, float hc_eps, float clamp_min,
                        float clamp_max, int32_t iter_times, void* x_next, void* y, float* post_out,
                        float* comb_frag, float* inv_rms, float* mixes, float* h_res_logits,
                        float* pre, void* workspace, size_t workspace_bytes, int32_t* status, int64_t T,
                        int32_t N, int32_t D, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MHC_AMD_H_ */
