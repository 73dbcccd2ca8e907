"""mhc_post of layer l fused with mhc_pre_clamp_sinkhorn of layer l+1 (forward).

Between two sublayers the reference's model code runs

    x_next = mhc_post(x, h_res, h_out, h_post)                (src/mhc_post.py:296-352)
    out    = mhc_pre_clamp_sinkhorn(x_next, phi, alpha, base, ...)
                                                  (src/mhc_pre_clamp_sinkhorn.py:857-971)

``mhc_post_pre_clamp_sinkhorn`` returns the same ``(x_next, out)`` from the
gfx950 entry point ``mhc_post_pre_fwd_ex``: for N = 4 bf16 where the pre
forward has its single pass (T >= 8192, D = 4096 or 7168..8192) that kernel
forms x_next from x and h_out itself (x read once, x_next written once and
never read back; outputs bit-identical to the two operators, x_next to
``mhc_post``), and like the pre forward it reports a timed-out wait through
a status word (RuntimeError at the next check); other N = 4 bf16 shapes with
D % 64 == 0 and D >= 256 run one kernel that reads x once, writes x_next once
and feeds it to the pre contraction (the y pass then reads x_next back);
other shapes run the two kernels in turn.
The reference has no fused operator; argument meanings, shapes, dtypes and
errors are those of the two operators it replaces.  With ``need_backward``
the dict carries inv_rms, mixes, h_res_logits and pre, and ``x_scaled`` is
None (the backward recomputes x_next * inv_rms).
"""

from __future__ import annotations

import torch

from . import _lib
from .mhc_post import _flatten_bsn
from .mhc_pre_clamp_sinkhorn import SINGLE_PASS_MIN_T, _check_params


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
    _lib.SINGLE_PASS.check(block=False)  # earlier calls' bounded waits, where finished
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
        # the shapes a single pass can take report its bounded waits into a
        # status word, as the pre forward's
        slot = status = None
        if (N == 4 and T >= SINGLE_PASS_MIN_T and xf.dtype == torch.bfloat16
                and phi_c.dtype == torch.bfloat16 and not torch.cuda.is_current_stream_capturing()):
            slot, status = _lib.SINGLE_PASS.acquire()
        with torch.cuda.device(dev):
            rc = lib.mhc_post_pre_fwd_ex(
                xf.data_ptr(), hres.data_ptr(), hout.data_ptr(), hpost.data_ptr(), xcode,
                phi_c.data_ptr(), pcode, alpha_c.data_ptr(), base_c.data_ptr(), float(norm_eps),
                float(hc_eps), float(clamp_min), float(clamp_max), int(iter_times),
                x_next.data_ptr(), y.data_ptr(), post_out.data_ptr(), comb.data_ptr(),
                _lib.ptr(inv_rms), _lib.ptr(mixes), _lib.ptr(logits), _lib.ptr(pre),
                ws.data_ptr(), ws_bytes, status, T, N, D, _lib.stream_of(xf))
        _lib.check(rc, "mhc_post_pre_clamp_sinkhorn")
        if slot is not None:
            _lib.SINGLE_PASS.commit(slot, torch.cuda.current_stream(dev))
    yshape = shape[:-2] + (D,)
    out = {"y": y.reshape(yshape), "post_out": post_out, "comb_frag": comb}
    if need_backward:
        out.update(inv_rms=inv_rms, x_scaled=None, mixes=mixes, h_res_logits=logits, pre=pre)
    return x_next.reshape(shape), out

