"""mhc_post: write the sublayer output back into the N residual streams.

    y[t, i, :] = sum_j h_res[t, j, i] * x[t, j, :] + h_post[t, i] * h_out[t, :]

Same contract as the reference operator (src/mhc_post.py:296-352): x is
(B, S, N, D) or (T, N, D), h_res (.., N, N), h_out (.., D), h_post (.., N);
the output has x's shape and dtype, accumulation is fp32.  ``mhc_post`` runs
the gfx950 kernel ``mhc_post_fwd`` of libmhc_amd.so; ``mhc_post_ref`` is the
pure-PyTorch reference of the same semantics.
"""

from __future__ import annotations

import torch

from . import _lib

SUPPORTED_N = (2, 4, 6, 8)


def _flatten_bsn(x, h_res, h_out, h_post):
    """(B,S,N,D) or (T,N,D) -> contiguous TND views plus the original shape
    (src/mhc_post.py:274-292)."""
    if x.dim() == 4:
        B, S, N, D = x.shape
        T = B * S
        return (x.reshape(T, N, D).contiguous(), h_res.reshape(T, N, N).contiguous(),
                h_out.reshape(T, D).contiguous(), h_post.reshape(T, N).contiguous(),
                (B, S, N, D))
    if x.dim() == 3:
        T, N, D = x.shape
        return (x.contiguous(), h_res.reshape(T, N, N).contiguous(),
                h_out.reshape(T, D).contiguous(), h_post.reshape(T, N).contiguous(), (T, N, D))
    raise ValueError(f"unsupported x.dim()={x.dim()}, expect 3 or 4")


def mhc_post(x, h_res, h_out, h_post):
    """Forward of mhc_post on the HIP device (no CPU fallback)."""
    _lib.require_device("mhc_post", x, h_res, h_out, h_post)
    xf, hres, hout, hpost, shape = _flatten_bsn(x, h_res, h_out, h_post)
    T, N, D = xf.shape
    if N not in SUPPORTED_N:
        raise NotImplementedError(f"mhc_post: N={N} not supported (supported: {SUPPORTED_N})")
    code = _lib.dtype_code("mhc_post", xf.dtype)
    hres = hres.to(torch.float32).contiguous()
    hpost = hpost.to(torch.float32).contiguous()
    hout = hout.to(xf.dtype).contiguous()
    out = torch.empty_like(xf)
    if T > 0:
        lib = _lib.load()
        with torch.cuda.device(xf.device):
            rc = lib.mhc_post_fwd(xf.data_ptr(), hres.data_ptr(), hout.data_ptr(),
                                  hpost.data_ptr(), out.data_ptr(), T, N, D, code,
                                  _lib.stream_of(xf))
        _lib.check(rc, "mhc_post")
    return out.reshape(shape)


def mhc_post_ref(x, h_res, h_out, h_post):
    """Pure-PyTorch reference (src/mhc_post.py:344-352): fp32 math, cast to
    x's dtype."""
    orig_dtype = x.dtype
    xf, hres, hout, hpost, shape = _flatten_bsn(x, h_res, h_out, h_post)
    mixed = torch.einsum("tji,tjd->tid", hres.float(), xf.float())
    y = mixed + hpost.float().unsqueeze(-1) * hout.float().unsqueeze(1)
    return y.to(orig_dtype).reshape(shape)
