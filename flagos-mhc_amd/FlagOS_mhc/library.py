"""torch.library registration of the mHC operators (namespace ``flagos_mhc``).

Registered ops (opaque to torch.compile, with shape functions for fake/meta
tensors and autograd formulas, so a compiled graph keeps them whole and
HIP-graph capture records their kernels on the current stream):

    torch.ops.flagos_mhc.mhc_post(x, h_res, h_out, h_post) -> y
    torch.ops.flagos_mhc.mhc_post_backward(grad_y, x, h_res, h_out, h_post)
        -> (grad_x, grad_h_res, grad_h_out, grad_h_post)
    torch.ops.flagos_mhc.mhc_post_backward_sum(grad_y, grad_y2, x, h_res, h_out,
        h_post) -> the same for the gradient grad_y + grad_y2
    torch.ops.flagos_mhc.mhc_pre_clamp_sinkhorn(x, phi, alpha, base, norm_eps,
        hc_eps, clamp_min, clamp_max, iter_times)
        -> (y, post_out, comb_frag, inv_rms, mixes, pre)
    torch.ops.flagos_mhc.mhc_pre_clamp_sinkhorn_backward(x, phi, alpha, base,
        inv_rms, mixes, pre, grad_y, grad_post_out, grad_comb_frag, norm_eps,
        hc_eps, clamp_min, clamp_max, iter_times)
        -> (grad_x, grad_phi, grad_alpha, grad_base)
    torch.ops.flagos_mhc.mhc_pre_clamp_sinkhorn_backward_acc(x, phi, alpha, base,
        inv_rms, mixes, pre, grad_y, grad_post_out, grad_comb_frag, grad_x_in,
        norm_eps, hc_eps, clamp_min, clamp_max, iter_times)
        -> (grad_x_in + grad_x, grad_phi, grad_alpha, grad_base)
    torch.ops.flagos_mhc.mhc_post_pre_clamp_sinkhorn(x, h_res, h_out, h_post,
        phi, alpha, base, norm_eps, hc_eps, clamp_min, clamp_max, iter_times)
        -> (x_next, y, post_out, comb_frag, inv_rms, mixes, pre)

The forward pre op also returns the fp32 inv_rms, mixes and pre its backward
needs; they are marked non-differentiable (likewise for the fused op).
``mhc_post_op``, ``mhc_pre_clamp_sinkhorn_op`` and
``mhc_post_pre_clamp_sinkhorn_op`` are the autograd-aware entry points with
the return conventions of ``mhc_post_fn`` / ``mhc_pre_clamp_sinkhorn_fn``
(src/autograd.py:14-87) and ``mhc_post_pre_clamp_sinkhorn_fn``.  The kernels allocate nothing outside torch's
allocator and call no host synchronisation, so they can be captured in a
HIP graph (``torch.cuda.graph``) after one eager warm-up call.
"""

from __future__ import annotations

import math
from typing import Tuple

import torch
from torch import Tensor

from .mhc_post import mhc_post
from .mhc_post_backward import mhc_post_backward, mhc_post_backward_sum, post_backward_sum_fused
from .mhc_post_pre import mhc_post_pre_clamp_sinkhorn
from .mhc_pre_clamp_sinkhorn import _pre_forward
from .mhc_pre_clamp_sinkhorn_backward import _pre_backward, mhc_pre_clamp_sinkhorn_backward

NAMESPACE = "flagos_mhc"


# ---- mhc_post ---------------------------------------------------------------

@torch.library.custom_op(f"{NAMESPACE}::mhc_post", mutates_args=())
def _post(x: Tensor, h_res: Tensor, h_out: Tensor, h_post: Tensor) -> Tensor:
    return mhc_post(x, h_res, h_out, h_post)


@_post.register_fake
def _post_fake(x, h_res, h_out, h_post):
    return torch.empty_like(x, memory_format=torch.contiguous_format)


@torch.library.custom_op(f"{NAMESPACE}::mhc_post_backward", mutates_args=())
def _post_bwd(grad_y: Tensor, x: Tensor, h_res: Tensor, h_out: Tensor,
              h_post: Tensor) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
    return tuple(mhc_post_backward(grad_y, x, h_res, h_out, h_post))


@_post_bwd.register_fake
def _post_bwd_fake(grad_y, x, h_res, h_out, h_post):
    out_shape = tuple(grad_y.shape[:-2]) + (grad_y.shape[-1],)
    return (grad_y.new_empty(grad_y.shape, dtype=x.dtype), h_res.new_empty(h_res.shape),
            h_out.new_empty(out_shape), h_post.new_empty(h_post.shape))


@torch.library.custom_op(f"{NAMESPACE}::mhc_post_backward_sum", mutates_args=())
def _post_bwd_sum(grad_y: Tensor, grad_y2: Tensor, x: Tensor, h_res: Tensor, h_out: Tensor,
                  h_post: Tensor) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
    return tuple(mhc_post_backward_sum(grad_y, grad_y2, x, h_res, h_out, h_post))


@_post_bwd_sum.register_fake
def _post_bwd_sum_fake(grad_y, grad_y2, x, h_res, h_out, h_post):
    return _post_bwd_fake(grad_y, x, h_res, h_out, h_post)


def _post_setup(ctx, inputs, output):
    ctx.save_for_backward(*inputs)


def _post_grad(ctx, grad_y):
    x, h_res, h_out, h_post = ctx.saved_tensors
    return torch.ops.flagos_mhc.mhc_post_backward(grad_y.contiguous(), x, h_res, h_out, h_post)


_post.register_autograd(_post_grad, setup_context=_post_setup)


# ---- mhc_pre_clamp_sinkhorn -------------------------------------------------

@torch.library.custom_op(f"{NAMESPACE}::mhc_pre_clamp_sinkhorn", mutates_args=())
def _pre(x: Tensor, phi: Tensor, alpha: Tensor, base: Tensor, norm_eps: float, hc_eps: float,
         clamp_min: float, clamp_max: float, iter_times: int,
         compensated: bool = False) -> Tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    # compensated only selects the backward's reductions
    out = _pre_forward(x, phi, alpha, base, norm_eps, hc_eps, clamp_min, clamp_max, iter_times,
                       need_backward=True, want_x_scaled=False)
    return (out["y"], out["post_out"], out["comb_frag"], out["inv_rms"], out["mixes"], out["pre"])


def _pre_dims(x):
    if x.dim() not in (3, 4):
        raise ValueError(f"unsupported x.dim()={x.dim()}")
    N, D = x.shape[-2], x.shape[-1]
    T = math.prod(x.shape[:-2])
    return T, N, D


@_pre.register_fake
def _pre_fake(x, phi, alpha, base, norm_eps, hc_eps, clamp_min, clamp_max, iter_times,
              compensated=False):
    T, N, D = _pre_dims(x)
    M = N * (N + 2)
    f32 = dict(dtype=torch.float32)
    return (x.new_empty(tuple(x.shape[:-2]) + (D,)), x.new_empty((T, N), **f32),
            x.new_empty((T, N, N), **f32), x.new_empty((T,), **f32), x.new_empty((T, M), **f32),
            x.new_empty((T, N), **f32))


@torch.library.custom_op(f"{NAMESPACE}::mhc_pre_clamp_sinkhorn_backward", mutates_args=())
def _pre_bwd(x: Tensor, phi: Tensor, alpha: Tensor, base: Tensor, inv_rms: Tensor, mixes: Tensor,
             pre: Tensor, grad_y: Tensor, grad_post_out: Tensor, grad_comb_frag: Tensor,
             norm_eps: float, hc_eps: float, clamp_min: float, clamp_max: float,
             iter_times: int, compensated: bool = False) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
    return tuple(mhc_pre_clamp_sinkhorn_backward(
        x, phi, alpha, base, inv_rms, None, mixes, None, pre, grad_y, grad_post_out,
        grad_comb_frag, norm_eps=norm_eps, hc_eps=hc_eps, clamp_min=clamp_min,
        clamp_max=clamp_max, iter_times=iter_times, compensated=compensated))


@_pre_bwd.register_fake
def _pre_bwd_fake(x, phi, alpha, base, inv_rms, mixes, pre, grad_y, grad_post_out,
                  grad_comb_frag, norm_eps, hc_eps, clamp_min, clamp_max, iter_times,
                  compensated=False):
    f32 = dict(dtype=torch.float32)
    return (x.new_empty(x.shape), phi.new_empty(phi.shape, **f32), alpha.new_empty((3,), **f32),
            base.new_empty((base.numel(),), **f32))


@torch.library.custom_op(f"{NAMESPACE}::mhc_pre_clamp_sinkhorn_backward_acc", mutates_args=())
def _pre_bwd_acc(x: Tensor, phi: Tensor, alpha: Tensor, base: Tensor, inv_rms: Tensor,
                 mixes: Tensor, pre: Tensor, grad_y: Tensor, grad_post_out: Tensor,
                 grad_comb_frag: Tensor, grad_x_in: Tensor, norm_eps: float, hc_eps: float,
                 clamp_min: float, clamp_max: float, iter_times: int,
                 compensated: bool = False) -> Tuple[Tensor, Tensor, Tensor, Tensor]:
    return tuple(_pre_backward(x, phi, alpha, base, inv_rms, mixes, pre, grad_y, grad_post_out,
                               grad_comb_frag, norm_eps, hc_eps, clamp_min, clamp_max, iter_times,
                               grad_x_in=grad_x_in, compensated=compensated))


@_pre_bwd_acc.register_fake
def _pre_bwd_acc_fake(x, phi, alpha, base, inv_rms, mixes, pre, grad_y, grad_post_out,
                      grad_comb_frag, grad_x_in, norm_eps, hc_eps, clamp_min, clamp_max, iter_times,
                      compensated=False):
    return _pre_bwd_fake(x, phi, alpha, base, inv_rms, mixes, pre, grad_y, grad_post_out,
                         grad_comb_frag, norm_eps, hc_eps, clamp_min, clamp_max, iter_times)


def _pre_setup(ctx, inputs, output):
    x, phi, alpha, base, norm_eps, hc_eps, clamp_min, clamp_max, iter_times, *opt = inputs
    _, _, _, inv_rms, mixes, pre = output
    ctx.mark_non_differentiable(inv_rms, mixes, pre)
    ctx.save_for_backward(x, phi, alpha, base, inv_rms, mixes, pre)
    ctx.args = (norm_eps, hc_eps, clamp_min, clamp_max, iter_times, bool(opt[0]) if opt else False)


def _pre_grad(ctx, grad_y, grad_post_out, grad_comb_frag, _g_inv, _g_mixes, _g_pre):
    x, phi, alpha, base, inv_rms, mixes, pre = ctx.saved_tensors
    gx, gphi, galpha, gbase = torch.ops.flagos_mhc.mhc_pre_clamp_sinkhorn_backward(
        x, phi, alpha, base, inv_rms, mixes, pre, grad_y.contiguous(), grad_post_out.contiguous(),
        grad_comb_frag.contiguous(), *ctx.args)
    return (gx, gphi.to(phi.dtype), galpha.reshape(alpha.shape).to(alpha.dtype),
            gbase.reshape(base.shape).to(base.dtype), None, None, None, None, None, None)


_pre.register_autograd(_pre_grad, setup_context=_pre_setup)


# ---- mhc_post (layer l) fused with mhc_pre_clamp_sinkhorn (layer l+1) --------

@torch.library.custom_op(f"{NAMESPACE}::mhc_post_pre_clamp_sinkhorn", mutates_args=())
def _post_pre(x: Tensor, h_res: Tensor, h_out: Tensor, h_post: Tensor, phi: Tensor, alpha: Tensor,
              base: Tensor, norm_eps: float, hc_eps: float, clamp_min: float, clamp_max: float,
              iter_times: int,
              compensated: bool = False) -> Tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    x_next, out = mhc_post_pre_clamp_sinkhorn(x, h_res, h_out, h_post, phi, alpha, base, norm_eps,
                                              hc_eps, clamp_min, clamp_max, iter_times,
                                              need_backward=True)
    return (x_next, out["y"], out["post_out"], out["comb_frag"], out["inv_rms"], out["mixes"],
            out["pre"])


@_post_pre.register_fake
def _post_pre_fake(x, h_res, h_out, h_post, phi, alpha, base, norm_eps, hc_eps, clamp_min,
                   clamp_max, iter_times, compensated=False):
    return (torch.empty_like(x, memory_format=torch.contiguous_format),) + tuple(
        _pre_fake(x, phi, alpha, base, norm_eps, hc_eps, clamp_min, clamp_max, iter_times))


def _post_pre_setup(ctx, inputs, output):
    x, h_res, h_out, h_post, phi, alpha, base, norm_eps, hc_eps, clamp_min, clamp_max, iter_times, *opt = inputs
    x_next, _, _, _, inv_rms, mixes, pre = output
    ctx.mark_non_differentiable(inv_rms, mixes, pre)
    ctx.save_for_backward(x, h_res, h_out, h_post, phi, alpha, base, x_next, inv_rms, mixes, pre)
    ctx.args = (norm_eps, hc_eps, clamp_min, clamp_max, iter_times, bool(opt[0]) if opt else False)


def _post_pre_grad(ctx, grad_x_next, grad_y, grad_post_out, grad_comb_frag, _g_inv, _g_mixes,
                   _g_pre):
    x, h_res, h_out, h_post, phi, alpha, base, x_next, inv_rms, mixes, pre = ctx.saved_tensors
    # as MhcPostPreClampSinkhornFn.backward: the post kernel reads both parts
    # of x_next's gradient where it has a summed form, else the pre backward
    # adds them
    N, D = x.shape[-2], x.shape[-1]
    if post_backward_sum_fused(x.numel() // (N * D), N, D, x.dtype):
        g, gphi, galpha, gbase = torch.ops.flagos_mhc.mhc_pre_clamp_sinkhorn_backward(
            x_next, phi, alpha, base, inv_rms, mixes, pre, grad_y.contiguous(),
            grad_post_out.contiguous(), grad_comb_frag.contiguous(), *ctx.args)
        gx, ghres, ghout, ghpost = torch.ops.flagos_mhc.mhc_post_backward_sum(
            grad_x_next.contiguous(), g, x, h_res, h_out, h_post)
    else:
        g, gphi, galpha, gbase = torch.ops.flagos_mhc.mhc_pre_clamp_sinkhorn_backward_acc(
            x_next, phi, alpha, base, inv_rms, mixes, pre, grad_y.contiguous(),
            grad_post_out.contiguous(), grad_comb_frag.contiguous(), grad_x_next.contiguous(), *ctx.args)
        gx, ghres, ghout, ghpost = torch.ops.flagos_mhc.mhc_post_backward(g, x, h_res, h_out, h_post)
    return (gx, ghres, ghout, ghpost, gphi.to(phi.dtype), galpha.reshape(alpha.shape).to(alpha.dtype),
            gbase.reshape(base.shape).to(base.dtype), None, None, None, None, None, None)


_post_pre.register_autograd(_post_pre_grad, setup_context=_post_pre_setup)


# ---- autograd-aware entry points ---------------------------------------------

def mhc_post_op(x, h_res, h_out, h_post):
    """``mhc_post`` through the registered op (differentiable, compilable)."""
    return torch.ops.flagos_mhc.mhc_post(x, h_res, h_out, h_post)


def mhc_pre_clamp_sinkhorn_op(x, phi, alpha, base, norm_eps=1e-6, hc_eps=1e-6, clamp_min=0.0,
                              clamp_max=0.0, iter_times=20, *, compensated=False):
    """``mhc_pre_clamp_sinkhorn`` through the registered op: (y, post_out,
    comb_frag), differentiable in x, phi, alpha and base; ``compensated``
    selects the backward's compensated T-reductions."""
    y, post_out, comb, _, _, _ = torch.ops.flagos_mhc.mhc_pre_clamp_sinkhorn(
        x, phi, alpha, base, float(norm_eps), float(hc_eps), float(clamp_min), float(clamp_max),
        int(iter_times), bool(compensated))
    return y, post_out, comb


def mhc_post_pre_clamp_sinkhorn_op(x, h_res, h_out, h_post, phi, alpha, base, norm_eps=1e-6,
                                   hc_eps=1e-6, clamp_min=0.0, clamp_max=0.0, iter_times=20, *,
                                   compensated=False):
    """The fused mhc_post + mhc_pre_clamp_sinkhorn through the registered op:
    (x_next, y, post_out, comb_frag), differentiable in every tensor input."""
    x_next, y, post_out, comb, _, _, _ = torch.ops.flagos_mhc.mhc_post_pre_clamp_sinkhorn(
        x, h_res, h_out, h_post, phi, alpha, base, float(norm_eps), float(hc_eps), float(clamp_min),
        float(clamp_max), int(iter_times), bool(compensated))
    return x_next, y, post_out, comb
