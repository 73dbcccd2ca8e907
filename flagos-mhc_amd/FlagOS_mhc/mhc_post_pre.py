"""mhc_post of layer l fused with mhc_pre_clamp_sinkhorn of layer l+1 (forward).

Between two sublayers the reference's model code runs

    x_next = mhc_post(x, h_res, h_out, h_post)                (src/mhc_post.py:296-352)
    out    = mhc_pre_clamp_sinkhorn(x_next, phi, alpha, base, ...)
                                                  (src/mhc_pre_clamp_sinkhorn.py:857-971)

``mhc_post_pre_clamp_sinkhorn`` returns the same ``(x_next, out)`` from the
gfx950 entry point ``mhc_post_pre_fwd``: for N = 4 bf16 with D % 64 == 0 and
D >= 256 one kernel reads x once, writes x_next once (bit-identical to
``mhc_post``) and feeds the same values to the pre contraction, saving one
full read of the residual streams (the y pass then reads x_next back); other
shapes run the two kernels in turn.
The reference has no fused operator; argument meanings, shapes, dtypes and
errors are those of the two operators it replaces.  With ``need_backward``
the dict carries inv_rms, mixes, h_res_logits and pre, and ``x_scaled`` is
None (the backward recomputes x_next * inv_rms).
"""

from __future__ import annotations

import torch

from . import _lib
from .mhc_post import _flatten_bsn
from .mhc_pre_clamp_sinkhorn import _check_params


def mhc_post_pre_clamp_sinkhorn(
    x: torch.Tensor,
    h_res: torch.Tensor,
    h_out: torch.Tensor,
    h_post: torch.Tensor,
    phi: torch.Tensor,
    alpha: torch.Tensor,
    base: torch.Tensor,
    norm_eps: float = 1e-6,
    hc_eps: float = 1e-6,
    clamp_min: float = 0.0,
    clamp_max: float = 0.0,
    iter_times: int = 20,
    need_backward: bool = False,
):
    """Returns (x_next, out): x_next shaped like x in x's dtype, out the dict of
    mhc_pre_clamp_sinkhorn(x_next, phi, alpha, base, ...)."""
    _lib.require_device("mhc_post_pre_clamp_sinkhorn", x, h_res, h_out, h_post, phi, alpha, base)
    xf, hres, hout, hpost, shape = _flatten_bsn(x, h_res, h_out, h_post)
    T, N, D = xf.shape
    M = _check_params(N, D, phi, alpha, base)
    xcode = _lib.dtype_code("mhc_post_pre_clamp_sinkhorn", xf.dtype)
    phi_c = phi.contiguous()
    pcode = _lib.dtype_code("mhc_post_pre_clamp_sinkhorn (phi)", phi_c.dtype)
    hres = hres.to(torch.float32).contiguous()
    hpost = hpost.to(torch.float32).contiguous()
    hout = hout.to(xf.dtype).contiguous()
    alpha_c = alpha.reshape(3).to(torch.float32).contiguous()
    base_c = base.reshape(M).to(torch.float32).contiguous()
    dev = xf.device
    f32 = dict(dtype=torch.float32, device=dev)

    x_next = torch.empty_like(xf)
    y = torch.empty((T, D), dtype=xf.dtype, device=dev)
    post_out = torch.empty((T, N), **f32)
    comb = torch.empty((T, N, N), **f32)
    inv_rms = mixes = logits = pre = None
    if need_backward:
        inv_rms = torch.empty((T,), **f32)
        mixes = torch.empty((T, M), **f32)
        logits = torch.empty((T, N, N), **f32)
        pre = torch.empty((T, N), **f32)
    if T > 0:
        lib = _lib.load()
        ws_bytes = int(lib.mhc_post_pre_fwd_workspace_size(T, N, D, pcode))
        ws = torch.empty((max(ws_bytes, 1),), dtype=torch.uint8, device=dev)
        with torch.cuda.device(dev):
            rc = lib.mhc_post_pre_fwd(
                xf.data_ptr(), hres.data_ptr(), hout.data_ptr(), hpost.data_ptr(), xcode,
                phi_c.data_ptr(), pcode, alpha_c.data_ptr(), base_c.data_ptr(), float(norm_eps),
                float(hc_eps), float(clamp_min), float(clamp_max), int(iter_times),
                x_next.data_ptr(), y.data_ptr(), post_out.data_ptr(), comb.data_ptr(),
                _lib.ptr(inv_rms), _lib.ptr(mixes), _lib.ptr(logits), _lib.ptr(pre),
                ws.data_ptr(), ws_bytes, T, N, D, _lib.stream_of(xf))
        _lib.check(rc, "mhc_post_pre_clamp_sinkhorn")
    yshape = shape[:-2] + (D,)
    out = {"y": y.reshape(yshape), "post_out": post_out, "comb_frag": comb}
    if need_backward:
        out.update(inv_rms=inv_rms, x_scaled=None, mixes=mixes, h_res_logits=logits, pre=pre)
    return x_next.reshape(shape), out

