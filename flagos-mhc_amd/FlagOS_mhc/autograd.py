"""torch.autograd.Function wrappers pairing each forward with its backward,
with the reference's contract (src/autograd.py:14-87)."""

from __future__ import annotations

import torch

from .mhc_post import mhc_post
from .mhc_post_backward import mhc_post_backward, mhc_post_backward_sum, post_backward_sum_fused
from .mhc_post_pre import mhc_post_pre_clamp_sinkhorn
from .mhc_pre_clamp_sinkhorn import _pre_forward
from .mhc_pre_clamp_sinkhorn_backward import _pre_backward, mhc_pre_clamp_sinkhorn_backward


class MhcPostFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, h_res, h_out, h_post):
        y = mhc_post(x, h_res, h_out, h_post)
        ctx.save_for_backward(x, h_res, h_out, h_post)
        return y

    @staticmethod
    def backward(ctx, grad_y):
        x, h_res, h_out, h_post = ctx.saved_tensors
        return mhc_post_backward(grad_y.contiguous(), x, h_res, h_out, h_post)


def mhc_post_fn(x, h_res, h_out, h_post):
    """Autograd-aware mhc_post."""
    return MhcPostFn.apply(x, h_res, h_out, h_post)


class MhcPreClampSinkhornFn(torch.autograd.Function):
    """Forward saves x, phi, alpha, base and the fp32 inv_rms / mixes / pre
    of the forward.  Unlike the reference it does not materialise the fp32
    x_scaled (4*N*D bytes per token): the backward recomputes x * inv_rms."""

    @staticmethod
    def forward(ctx, x, phi, alpha, base, norm_eps, hc_eps, clamp_min, clamp_max, iter_times,
                compensated=False):
        out = _pre_forward(x, phi, alpha, base, norm_eps, hc_eps, clamp_min, clamp_max,
                           iter_times, need_backward=True, want_x_scaled=False)
        ctx.save_for_backward(x, phi, alpha, base, out["inv_rms"], out["mixes"], out["pre"])
        ctx.norm_eps = norm_eps
        ctx.hc_eps = hc_eps
        ctx.clamp_min = clamp_min
        ctx.clamp_max = clamp_max
        ctx.iter_times = iter_times
        ctx.compensated = bool(compensated)
        return out["y"], out["post_out"], out["comb_frag"]

    @staticmethod
    def backward(ctx, grad_y, grad_post_out, grad_comb_frag):
        x, phi, alpha, base, inv_rms, mixes, pre = ctx.saved_tensors
        # an output that did not reach the loss arrives as None: its gradient is zero
        if grad_y is None:
            grad_y = torch.zeros(x.shape[:-2] + x.shape[-1:], dtype=x.dtype, device=x.device)
        if grad_post_out is None:
            grad_post_out = torch.zeros_like(pre)
        if grad_comb_frag is None:
            N = pre.shape[-1]
            grad_comb_frag = torch.zeros((pre.shape[0], N, N), dtype=torch.float32, device=pre.device)
        gx, gphi, galpha, gbase = mhc_pre_clamp_sinkhorn_backward(
            x, phi, alpha, base, inv_rms, None, mixes, None, pre,
            grad_y.contiguous(), grad_post_out.contiguous(), grad_comb_frag.contiguous(),
            norm_eps=ctx.norm_eps, hc_eps=ctx.hc_eps, clamp_min=ctx.clamp_min,
            clamp_max=ctx.clamp_max, iter_times=ctx.iter_times, compensated=ctx.compensated)
        # (x, phi, alpha, base, norm_eps, hc_eps, clamp_min, clamp_max, iter_times, compensated)
        return gx, gphi, galpha, gbase, None, None, None, None, None, None


def mhc_pre_clamp_sinkhorn_fn(
    x, phi, alpha, base,
    norm_eps=1e-6, hc_eps=1e-6,
    clamp_min=0.0, clamp_max=0.0,
    iter_times=20,
    *,
    compensated=False,
):
    """Autograd-aware mhc_pre_clamp_sinkhorn. Returns (y, post_out, comb_frag).
    ``compensated`` (beyond the reference) selects the backward's compensated
    T-reductions (see mhc_pre_clamp_sinkhorn_backward)."""
    return MhcPreClampSinkhornFn.apply(
        x, phi, alpha, base, norm_eps, hc_eps, clamp_min, clamp_max, iter_times, compensated)


class MhcPostPreClampSinkhornFn(torch.autograd.Function):
    """mhc_post (layer l) + mhc_pre_clamp_sinkhorn (layer l+1) with one fused
    forward.  The backward runs the pre backward on x_next, then the post
    backward for x_next's whole gradient: the post kernel reads the pre
    backward's grad_x beside the gradient that reaches x_next directly
    (``mhc_post_bwd_sum``).  Where the post kernel for the shape has no
    summed form (N = 4 bf16, D < 2048), the pre backward adds that gradient
    into its grad_x instead (``mhc_pre_bwd_acc``)."""

    @staticmethod
    def forward(ctx, x, h_res, h_out, h_post, phi, alpha, base, norm_eps, hc_eps, clamp_min,
                clamp_max, iter_times, compensated=False):
        x_next, out = mhc_post_pre_clamp_sinkhorn(
            x, h_res, h_out, h_post, phi, alpha, base, norm_eps, hc_eps, clamp_min, clamp_max,
            iter_times, need_backward=True)
        ctx.save_for_backward(x, h_res, h_out, h_post, phi, alpha, base, x_next, out["inv_rms"],
                              out["mixes"], out["pre"])
        ctx.args = (norm_eps, hc_eps, clamp_min, clamp_max, iter_times)
        ctx.compensated = bool(compensated)
        return x_next, out["y"], out["post_out"], out["comb_frag"]

    @staticmethod
    def backward(ctx, grad_x_next, grad_y, grad_post_out, grad_comb_frag):
        x, h_res, h_out, h_post, phi, alpha, base, x_next, inv_rms, mixes, pre = ctx.saved_tensors
        norm_eps, hc_eps, clamp_min, clamp_max, iter_times = ctx.args
        if grad_y is None:
            grad_y = torch.zeros(x_next.shape[:-2] + x_next.shape[-1:], dtype=x.dtype, device=x.device)
        if grad_post_out is None:
            grad_post_out = torch.zeros_like(pre)
        if grad_comb_frag is None:
            N = pre.shape[-1]
            grad_comb_frag = torch.zeros((pre.shape[0], N, N), dtype=torch.float32, device=pre.device)
        N, D = x.shape[-2], x.shape[-1]
        use_sum = grad_x_next is not None and post_backward_sum_fused(x.numel() // (N * D), N, D, x.dtype)
        g, gphi, galpha, gbase = _pre_backward(
            x_next, phi, alpha, base, inv_rms, mixes, pre, grad_y.contiguous(),
            grad_post_out.contiguous(), grad_comb_frag.contiguous(), norm_eps, hc_eps, clamp_min,
            clamp_max, iter_times, grad_x_in=None if use_sum else grad_x_next,
            compensated=ctx.compensated)
        if use_sum:
            gx, ghres, ghout, ghpost = mhc_post_backward_sum(grad_x_next, g, x, h_res, h_out, h_post)
        else:
            gx, ghres, ghout, ghpost = mhc_post_backward(g, x, h_res, h_out, h_post)
        return gx, ghres, ghout, ghpost, gphi, galpha, gbase, None, None, None, None, None, None


def mhc_post_pre_clamp_sinkhorn_fn(
    x, h_res, h_out, h_post, phi, alpha, base,
    norm_eps=1e-6, hc_eps=1e-6,
    clamp_min=0.0, clamp_max=0.0,
    iter_times=20,
    *,
    compensated=False,
):
    """Autograd-aware fused mhc_post + mhc_pre_clamp_sinkhorn.  Returns
    (x_next, y, post_out, comb_frag); ``compensated`` as in
    mhc_pre_clamp_sinkhorn_fn."""
    return MhcPostPreClampSinkhornFn.apply(
        x, h_res, h_out, h_post, phi, alpha, base, norm_eps, hc_eps, clamp_min, clamp_max,
        iter_times, compensated)
