"""mhc_post_backward: the four vector-Jacobian products of mhc_post.

    grad_x[t,j,:]     = sum_i h_res[t,j,i] * grad_y[t,i,:]
    grad_h_res[t,j,i] = <x[t,j,:], grad_y[t,i,:]>
    grad_h_out[t,:]   = sum_i h_post[t,i] * grad_y[t,i,:]
    grad_h_post[t,i]  = <h_out[t,:], grad_y[t,i,:]>

Contract of the reference operator (src/mhc_post_backward.py:564-643):
grad_y (B,S,N,D) or (T,N,D); returns (grad_x shaped like grad_y,
grad_h_res shaped like h_res, grad_h_out (B,S,D) or (T,D), grad_h_post
shaped like h_post).  Output dtypes follow the reference operator's
``empty_like`` allocations: grad_x like x, grad_h_out like h_out, grad_h_res
and grad_h_post like their gates.  One gfx950 kernel computes all four in a
single pass with deterministic per-token reductions.
"""

from __future__ import annotations

import torch

from . import _lib
from .mhc_post import SUPPORTED_N


def _flatten(grad_y, x, h_res, h_out, h_post):
    """src/mhc_post_backward.py:564-590."""
    if grad_y.dim() == 4:
        B, S, N, D = grad_y.shape
        T = B * S
        return (grad_y.reshape(T, N, D).contiguous(), x.reshape(T, N, D).contiguous(),
                h_res.reshape(T, N, N).contiguous(), h_out.reshape(T, D).contiguous(),
                h_post.reshape(T, N).contiguous(), (B, S, N, D), (B, S, D))
    if grad_y.dim() == 3:
        T, N, D = grad_y.shape
        return (grad_y.contiguous(), x.contiguous(), h_res.reshape(T, N, N).contiguous(),
                h_out.reshape(T, D).contiguous(), h_post.reshape(T, N).contiguous(),
                (T, N, D), (T, D))
    raise ValueError(f"unsupported grad_y.dim()={grad_y.dim()}")


def mhc_post_backward(grad_y, x, h_res, h_out, h_post):
    """Backward of mhc_post on the HIP device (no CPU fallback)."""
    return _post_backward("mhc_post_backward", grad_y, None, x, h_res, h_out, h_post)


def mhc_post_backward_sum(grad_y, grad_y2, x, h_res, h_out, h_post):
    """mhc_post_backward for the incoming gradient grad_y + grad_y2 (same
    shape and dtype, added in fp32 inside the kernel as they are read).  Not
    part of the reference's API: the fused post + pre layer's backward uses it
    so that the pre backward's grad_x and the gradient reaching x_next
    directly are never summed into a tensor of their own."""
    if grad_y2.shape != grad_y.shape:
        raise ValueError(f"mhc_post_backward_sum: grad_y2 shape {tuple(grad_y2.shape)} "
                         f"!= grad_y shape {tuple(grad_y.shape)}")
    return _post_backward("mhc_post_backward_sum", grad_y, grad_y2, x, h_res, h_out, h_post)


def post_backward_sum_fused(T: int, N: int, D: int, dtype: torch.dtype) -> bool:
    """True when mhc_post_backward_sum runs the kernel form mhc_post_backward
    would for this shape (one more read, no slower form)."""
    return bool(_lib.load().mhc_post_bwd_sum_fused(T, N, D, _lib.dtype_code("mhc_post_backward_sum", dtype)))


def _post_backward(what, grad_y, grad_y2, x, h_res, h_out, h_post):
    _lib.require_device(what, grad_y, x, h_res, h_out, h_post, grad_y2)
    gy, xf, hres, hout, hpost, shape4, shape_out = _flatten(grad_y, x, h_res, h_out, h_post)
    T, N, D = gy.shape
    if N not in SUPPORTED_N:
        raise NotImplementedError(f"{what}: N={N} not supported (supported: {SUPPORTED_N})")
    code = _lib.dtype_code(what, xf.dtype)
    gy = gy.to(xf.dtype).contiguous()
    gy2 = None if grad_y2 is None else grad_y2.reshape(T, N, D).to(xf.dtype).contiguous()
    hout_k = hout.to(xf.dtype).contiguous()
    hres_k = hres.to(torch.float32).contiguous()
    hpost_k = hpost.to(torch.float32).contiguous()

    grad_x = torch.empty_like(xf)
    grad_hout = torch.empty((T, D), dtype=xf.dtype, device=xf.device)
    grad_hres = torch.empty((T, N, N), dtype=torch.float32, device=xf.device)
    grad_hpost = torch.empty((T, N), dtype=torch.float32, device=xf.device)
    if T > 0:
        lib = _lib.load()
        with torch.cuda.device(xf.device):
            tail = (hres_k.data_ptr(), hout_k.data_ptr(), hpost_k.data_ptr(), grad_x.data_ptr(),
                    grad_hres.data_ptr(), grad_hout.data_ptr(), grad_hpost.data_ptr(), T, N, D, code,
                    _lib.stream_of(xf))
            if gy2 is None:
                rc = lib.mhc_post_bwd(gy.data_ptr(), xf.data_ptr(), *tail)
            else:
                rc = lib.mhc_post_bwd_sum(gy.data_ptr(), gy2.data_ptr(), xf.data_ptr(), *tail)
        _lib.check(rc, what)
    return (
        grad_x.reshape(shape4),
        grad_hres.to(h_res.dtype).reshape(h_res.shape),
        grad_hout.to(h_out.dtype).reshape(shape_out),
        grad_hpost.to(h_post.dtype).reshape(h_post.shape),
    )


def mhc_post_backward_ref(grad_y, x, h_res, h_out, h_post):
    """Pure-PyTorch reference (src/mhc_post_backward.py:624-643): fp32 math;
    grad_x and grad_h_out cast to x's dtype, grad_h_res / grad_h_post fp32."""
    orig_dtype = x.dtype
    gy, xf, hres, hout, hpost, shape4, shape_out = _flatten(grad_y, x, h_res, h_out, h_post)
    gy32, x32 = gy.float(), xf.float()
    grad_x = torch.einsum("tji,tid->tjd", hres.float(), gy32).to(orig_dtype)
    grad_hres = torch.einsum("tjd,tid->tji", x32, gy32)
    grad_hout = torch.einsum("ti,tid->td", hpost.float(), gy32).to(orig_dtype)
    grad_hpost = torch.einsum("td,tid->ti", hout.float(), gy32)
    return (grad_x.reshape(shape4), grad_hres.reshape(h_res.shape),
            grad_hout.reshape(shape_out), grad_hpost.reshape(h_post.shape))
