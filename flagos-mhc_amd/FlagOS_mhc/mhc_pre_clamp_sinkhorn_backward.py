"""mhc_pre_clamp_sinkhorn_backward: gradients of the pre operator with respect
to x, phi, alpha and base, for upstream grad_y (of y), grad_post_out and
grad_comb_frag.

Semantics: torch autograd through the fp32 forward, as the reference's
mhc_pre_clamp_sinkhorn_backward_ref (src/mhc_pre_clamp_sinkhorn_backward.py:
1397-1453): clamp gradient passes where clamp_min <= logit <= clamp_max.

The gfx950 path (``mhc_pre_bwd``) takes the forward's saved inv_rms, mixes
and pre, recomputes the Sinkhorn states per token in registers, and writes
grad_x once:
    grad_x = grad_y * pre[n] + inv * (grad_mixes @ phi) + scale * x,
    scale  = -inv^2 * <grad_mixes, mixes> / (N*D).
grad_phi = (grad_mixes * inv)^T @ x runs on MFMA split over token ranges and
is reduced in a fixed order, as are grad_alpha and grad_base, so the result
is deterministic.  The reference's x_scaled and h_res_logits arguments are
accepted and not needed (x * inv_rms and the logits are recomputed), so
passing None is fine.

``compensated=True`` (keyword, beyond the reference's signature) selects the
compensated T-reductions of the production AscendC operator's deterministic
mode, which the reference lists as not replicated (README.md:197-204):
grad_phi from exact 16-token products added with Neumaier's compensation
(``mhc_pre_bwd_ex`` with ``MHC_PRE_BWD_COMPENSATED``), grad_alpha / grad_base
likewise; grad_x is unchanged.  It costs one more read of x.
"""

from __future__ import annotations

import torch

from . import _lib
from .mhc_pre_clamp_sinkhorn import SINGLE_PASS_MIN_T, SUPPORTED_N, _flatten


def mhc_pre_clamp_sinkhorn_backward(
    x: torch.Tensor,
    phi: torch.Tensor,
    alpha: torch.Tensor,
    base: torch.Tensor,
    inv_rms: torch.Tensor,
    x_scaled,
    mixes: torch.Tensor,
    h_res_logits,
    pre: torch.Tensor,
    grad_y: torch.Tensor,
    grad_post_out: torch.Tensor,
    grad_comb_frag: torch.Tensor,
    norm_eps: float = 1e-6,
    hc_eps: float = 1e-6,
    clamp_min: float = 0.0,
    clamp_max: float = 0.0,
    iter_times: int = 20,
    *,
    compensated: bool = False,
):
    """Returns (grad_x shaped like x in x's dtype, grad_phi (M, N*D) fp32,
    grad_alpha (3,) fp32, grad_base (M,) fp32)
    (src/mhc_pre_clamp_sinkhorn_backward.py:1292-1391)."""
    del x_scaled, h_res_logits  # recomputed
    return _pre_backward(x, phi, alpha, base, inv_rms, mixes, pre, grad_y, grad_post_out,
                         grad_comb_frag, norm_eps, hc_eps, clamp_min, clamp_max, iter_times,
                         compensated=compensated)


def _pre_backward(x, phi, alpha, base, inv_rms, mixes, pre, grad_y, grad_post_out, grad_comb_frag,
                  norm_eps, hc_eps, clamp_min, clamp_max, iter_times, grad_x_in=None,
                  compensated=False, single_pass=None):
    """mhc_pre_clamp_sinkhorn_backward (``mhc_pre_bwd_ex``); with ``grad_x_in``
    (shaped and typed like x) the returned grad_x is grad_x_in + dL/dx,
    accumulated inside the kernel; ``compensated`` selects the compensated
    T-reductions.  ``single_pass``: None lets the library choose (the
    single-pass form wherever it applies: N = 4 bf16, D = 4096 or 7168..8192,
    T >= 8192), False keeps the two-pass forms, True asks for the single pass
    explicitly."""
    del norm_eps  # folded into inv_rms
    _lib.require_device("mhc_pre_clamp_sinkhorn_backward", x, phi, alpha, base, inv_rms, mixes,
                        pre, grad_y, grad_post_out, grad_comb_frag, grad_x_in)
    # a forward whose single pass gave up a bounded wait left NaN inputs for
    # this call: raise here rather than propagate them
    _lib.SINGLE_PASS.check(block=True)
    if x.dim() not in (3, 4):
        raise ValueError(f"unsupported x.dim()={x.dim()}")
    shape = tuple(x.shape)
    xf, _ = _flatten(x)
    T, N, D = xf.shape
    if grad_y.dim() == 3:
        _B, _S, _D = grad_y.shape
        assert _B * _S == T and _D == D
    elif grad_y.dim() == 2:
        assert tuple(grad_y.shape) == (T, D)
    else:
        raise ValueError(f"unsupported grad_y.dim()={grad_y.dim()}")
    assert N in SUPPORTED_N, f"hc_mult={N} not supported (supported: {SUPPORTED_N})"
    M = N * (N + 2)
    assert tuple(phi.shape) == (M, N * D), f"phi shape {tuple(phi.shape)} != {(M, N * D)}"
    xcode = _lib.dtype_code("mhc_pre_clamp_sinkhorn_backward", xf.dtype)
    phi_c = phi.contiguous()
    pcode = _lib.dtype_code("mhc_pre_clamp_sinkhorn_backward (phi)", phi_c.dtype)
    dev = xf.device
    f32 = dict(dtype=torch.float32, device=dev)

    gy = grad_y.reshape(T, D).to(xf.dtype).contiguous()
    gpost = grad_post_out.reshape(T, N).to(torch.float32).contiguous()
    gcomb = grad_comb_frag.reshape(T, N, N).to(torch.float32).contiguous()
    inv_c = inv_rms.reshape(T).to(torch.float32).contiguous()
    mixes_c = mixes.reshape(T, M).to(torch.float32).contiguous()
    pre_c = pre.reshape(T, N).to(torch.float32).contiguous()
    alpha_c = alpha.reshape(3).to(torch.float32).contiguous()
    base_c = base.reshape(M).to(torch.float32).contiguous()

    grad_x = torch.empty((T, N * D), dtype=xf.dtype, device=dev)
    grad_phi = torch.empty((M, N * D), **f32)
    grad_alpha = torch.empty((3,), **f32)
    grad_base = torch.empty((M,), **f32)
    lib = _lib.load()
    ws_bytes = int(lib.mhc_pre_bwd_workspace_size(T, N, D, pcode, int(iter_times)))
    ws = torch.empty((max(ws_bytes, 1),), dtype=torch.uint8, device=dev)
    common = (xf.data_ptr(), xcode, phi_c.data_ptr(), pcode, alpha_c.data_ptr(), base_c.data_ptr(),
              inv_c.data_ptr(), mixes_c.data_ptr(), pre_c.data_ptr(), gy.data_ptr(),
              gpost.data_ptr(), gcomb.data_ptr(), float(hc_eps), float(clamp_min),
              float(clamp_max), int(iter_times))
    gin = None if grad_x_in is None else grad_x_in.reshape(T, N * D).to(xf.dtype).contiguous()
    flags = _lib.PRE_BWD_COMPENSATED if compensated else 0
    if single_pass is not None:
        flags |= _lib.PRE_BWD_SINGLE_PASS if single_pass else _lib.PRE_BWD_TWO_PASS
    # the shapes the single-pass form can take (N = 4, bf16, T >= 8192, no
    # grad_x_in, not compensated; never under stream capture) report its
    # bounded waits into a status word
    slot = status = None
    if (single_pass is not False and N == 4 and T >= SINGLE_PASS_MIN_T and xf.dtype == torch.bfloat16
            and phi_c.dtype == torch.bfloat16 and gin is None and not compensated
            and not torch.cuda.is_current_stream_capturing()):
        slot, status = _lib.SINGLE_PASS.acquire()
    with torch.cuda.device(dev):
        rc = lib.mhc_pre_bwd_ex(*common, _lib.ptr(gin), grad_x.data_ptr(), grad_phi.data_ptr(),
                                grad_alpha.data_ptr(), grad_base.data_ptr(), flags, status,
                                ws.data_ptr(), ws_bytes, T, N, D, _lib.stream_of(xf))
    _lib.check(rc, "mhc_pre_clamp_sinkhorn_backward")
    if slot is not None:
        _lib.SINGLE_PASS.commit(slot, torch.cuda.current_stream(dev))
    return grad_x.view(*shape), grad_phi.reshape(phi.shape), grad_alpha, grad_base


def mhc_pre_clamp_sinkhorn_backward_ref(
    x, phi, alpha, base,
    grad_y, grad_post_out, grad_comb_frag,
    norm_eps=1e-6, hc_eps=1e-6,
    clamp_min=0.0, clamp_max=0.0,
    iter_times=20,
):
    """Pure-PyTorch reference: autograd through an fp32 restatement of the
    forward for the loss <grad_y, y> + <grad_post_out, post_out> +
    <grad_comb_frag, comb_frag> (src/mhc_pre_clamp_sinkhorn_backward.py:
    1397-1453).  Returns (grad_x in x's dtype, grad_phi, grad_alpha,
    grad_base) fp32."""
    orig_dtype = x.dtype
    leaves = [t.detach().to(torch.float32).requires_grad_(True) for t in (x, phi, alpha, base)]
    x_, phi_, a, b = leaves
    xf = x_.reshape(-1, x_.shape[-2], x_.shape[-1])
    T, N, D = xf.shape
    x32 = xf.reshape(T, N * D)
    inv = torch.rsqrt(x32.pow(2).mean(dim=-1, keepdim=True) + norm_eps)
    mixes = (x32 * inv) @ phi_.t()
    pre = torch.sigmoid(mixes[:, :N] * a[0] + b[:N]) + hc_eps
    post_out = 2.0 * torch.sigmoid(mixes[:, N:2 * N] * a[1] + b[N:2 * N])
    logits = (mixes[:, 2 * N:] * a[2] + b[2 * N:]).reshape(T, N, N)
    lc = torch.clamp(logits, clamp_min, clamp_max) if (clamp_min != 0.0 or clamp_max != 0.0) else logits
    e = (lc - lc.max(dim=-1, keepdim=True).values).exp()
    comb = e / e.sum(dim=-1, keepdim=True) + hc_eps
    comb = comb / (comb.sum(dim=-2, keepdim=True) + hc_eps)
    for _ in range(iter_times - 1):
        comb = comb / (comb.sum(dim=-1, keepdim=True) + hc_eps)
        comb = comb / (comb.sum(dim=-2, keepdim=True) + hc_eps)
    y = (xf * pre.unsqueeze(-1)).sum(dim=-2)
    loss = ((y * grad_y.to(torch.float32).reshape(T, D)).sum()
            + (post_out * grad_post_out.to(torch.float32).reshape(T, N)).sum()
            + (comb * grad_comb_frag.to(torch.float32).reshape(T, N, N)).sum())
    dx, dphi, da, db = torch.autograd.grad(loss, leaves)
    return dx.to(orig_dtype), dphi, da, db
