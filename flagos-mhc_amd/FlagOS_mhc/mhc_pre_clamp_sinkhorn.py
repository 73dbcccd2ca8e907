"""mhc_pre_clamp_sinkhorn: mix the N residual streams into the sublayer input.

Pipeline (semantics of the reference's mhc_pre_clamp_sinkhorn_ref,
src/mhc_pre_clamp_sinkhorn.py:974-1022):

1. inv_rms = rsqrt(mean(x[t]^2 over N*D) + norm_eps)
2. mixes   = (x[t] * inv_rms) @ phi^T                      (T, M), M = 2N + N^2
3. pre      = sigmoid(mixes[:, :N] * alpha[0] + base[:N]) + hc_eps
   post_out = 2 * sigmoid(mixes[:, N:2N] * alpha[1] + base[N:2N])
   logits   = mixes[:, 2N:] * alpha[2] + base[2N:]         (T, N, N)
4. clamp(logits, clamp_min, clamp_max) iff clamp_min != 0 or clamp_max != 0,
   row softmax, + hc_eps, column normalisation, then iter_times - 1
   (row, column) normalisations, every denominator being sum + hc_eps
5. y = sum_n x[:, n, :] * pre[:, n]                        (B,S,D) or (T,D)

``mhc_pre_clamp_sinkhorn`` runs all five stages in one gfx950 kernel
(``mhc_pre_fwd``): the N*D -> M contraction on bf16 MFMA with fp32
accumulation, the Sinkhorn stage in registers.  It returns the reference's
dict; with ``need_backward=True`` also inv_rms, x_scaled, mixes,
h_res_logits (pre-clamp) and pre.
"""

from __future__ import annotations

import torch

from . import _lib

SUPPORTED_N = (4, 8)
SINGLE_PASS_MIN_T = 8192  # fewest tokens the single-pass forms take (csrc/pre_fwd_coop.hpp, pre_bwd_coop.hpp)


def _flatten(x):
    """(B,S,N,D) or (T,N,D) -> (contiguous TND, shape of y)
    (src/mhc_pre_clamp_sinkhorn.py:844-854)."""
    if x.dim() == 4:
        B, S, N, D = x.shape
        return x.reshape(B * S, N, D).contiguous(), (B, S, D)
    if x.dim() == 3:
        T, N, D = x.shape
        return x.contiguous(), (T, D)
    raise ValueError(f"unsupported x.dim()={x.dim()}")


def _check_params(N, D, phi, alpha, base):
    hc_mix = N * (N + 2)
    assert N in SUPPORTED_N, f"hc_mult={N} not supported (supported: {SUPPORTED_N})"
    assert tuple(phi.shape) == (hc_mix, N * D), f"phi shape {tuple(phi.shape)} != {(hc_mix, N * D)}"
    assert alpha.numel() == 3
    assert base.numel() == hc_mix
    return hc_mix


def _pre_forward(x, phi, alpha, base, norm_eps, hc_eps, clamp_min, clamp_max, iter_times,
                 need_backward, want_x_scaled):
    _lib.require_device("mhc_pre_clamp_sinkhorn", x, phi, alpha, base)
    _lib.SINGLE_PASS.check(block=False)  # earlier calls' bounded waits, where finished
    xf, yshape = _flatten(x)
    T, N, D = xf.shape
    M = _check_params(N, D, phi, alpha, base)
    xcode = _lib.dtype_code("mhc_pre_clamp_sinkhorn", xf.dtype)
    phi_c = phi.contiguous()
    pcode = _lib.dtype_code("mhc_pre_clamp_sinkhorn (phi)", phi_c.dtype)
    alpha_c = alpha.reshape(3).to(torch.float32).contiguous()
    base_c = base.reshape(M).to(torch.float32).contiguous()
    dev = xf.device
    f32 = dict(dtype=torch.float32, device=dev)

    y = torch.empty((T, D), dtype=xf.dtype, device=dev)
    post_out = torch.empty((T, N), **f32)
    comb = torch.empty((T, N, N), **f32)
    inv_rms = mixes = logits = pre = x_scaled = None
    if need_backward:
        inv_rms = torch.empty((T,), **f32)
        mixes = torch.empty((T, M), **f32)
        logits = torch.empty((T, N, N), **f32)
        pre = torch.empty((T, N), **f32)
        if want_x_scaled:
            x_scaled = torch.empty((T, N * D), **f32)
    if T > 0:
        lib = _lib.load()
        ws_bytes = int(lib.mhc_pre_fwd_workspace_size(T, N, D, pcode))
        ws = torch.empty((max(ws_bytes, 1),), dtype=torch.uint8, device=dev)
        # the shapes the single-pass form can take (N = 4, bf16, T >= 8192;
        # never under stream capture) report its bounded waits into a status word
        slot = status = None
        if (N == 4 and T >= SINGLE_PASS_MIN_T and xf.dtype == torch.bfloat16
                and phi_c.dtype == torch.bfloat16 and not torch.cuda.is_current_stream_capturing()):
            slot, status = _lib.SINGLE_PASS.acquire()
        stream = _lib.stream_of(xf)
        with torch.cuda.device(dev):
            rc = lib.mhc_pre_fwd_ex(
                xf.data_ptr(), xcode, phi_c.data_ptr(), pcode, alpha_c.data_ptr(),
                base_c.data_ptr(), float(norm_eps), float(hc_eps), float(clamp_min),
                float(clamp_max), int(iter_times), y.data_ptr(), post_out.data_ptr(),
                comb.data_ptr(), _lib.ptr(inv_rms), _lib.ptr(mixes), _lib.ptr(logits),
                _lib.ptr(pre), _lib.ptr(x_scaled), ws.data_ptr(), ws_bytes, status, T, N, D,
                stream)
        _lib.check(rc, "mhc_pre_clamp_sinkhorn")
        if slot is not None:
            _lib.SINGLE_PASS.commit(slot, torch.cuda.current_stream(dev))
    result = {"y": y.reshape(yshape), "post_out": post_out, "comb_frag": comb}
    if need_backward:
        result.update(inv_rms=inv_rms, x_scaled=x_scaled, mixes=mixes, h_res_logits=logits,
                      pre=pre)
    return result


def mhc_pre_clamp_sinkhorn(
    x: torch.Tensor,
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
    """Fused mHC pre + clamp + Sinkhorn forward on the HIP device.

    Returns a dict with y (B,S,D)/(T,D) in x's dtype, post_out (T,N) and
    comb_frag (T,N,N) fp32; with need_backward=True also inv_rms (T,),
    x_scaled (T,N*D), mixes (T,M), h_res_logits (T,N,N) and pre (T,N), fp32
    (src/mhc_pre_clamp_sinkhorn.py:857-971).
    """
    return _pre_forward(x, phi, alpha, base, norm_eps, hc_eps, clamp_min, clamp_max,
                        iter_times, need_backward, want_x_scaled=True)


def mhc_pre_clamp_sinkhorn_ref(
    x, phi, alpha, base,
    norm_eps=1e-6, hc_eps=1e-6,
    clamp_min=0.0, clamp_max=0.0,
    iter_times=20,
):
    """Pure-PyTorch fp32 reference (src/mhc_pre_clamp_sinkhorn.py:974-1022).

    Returns y, post_out, comb_frag, inv_rms, mixes, h_res_logits, pre.
    """
    orig_dtype = x.dtype
    xf, yshape = _flatten(x)
    T, N, D = xf.shape
    x32 = xf.reshape(T, N * D).float()
    inv = torch.rsqrt(x32.pow(2).mean(dim=-1, keepdim=True) + norm_eps)
    mixes = (x32 * inv) @ phi.float().t()
    a, b = alpha.float(), base.float()
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
    y = (xf.float() * pre.unsqueeze(-1)).sum(dim=-2).to(orig_dtype)
    return {
        "y": y.reshape(yshape),
        "post_out": post_out,
        "comb_frag": comb,
        "inv_rms": inv.squeeze(-1),
        "mixes": mixes,
        "h_res_logits": logits,
        "pre": pre,
    }
