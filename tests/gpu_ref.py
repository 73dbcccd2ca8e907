"""Full-size references on the GPU for the parity tests (test infrastructure).

At the BASELINE config-5 shape (N=4, D=7168, T=65536) one activation tensor
holds 1.9e9 elements, too many to send through float64 numpy on the host.
These helpers keep the big contractions on the device in float64 (torch
matmuls and elementwise products in chunks of tokens) and take every
per-token nonlinearity (sigmoid heads, clamp, softmax, Sinkhorn and its VJP)
from the float64 oracle on the CPU, whose inputs there are only (T, M) and
(T, N, N) arrays.  The result is a float64 reference of the pre backward's
T-reductions (grad_phi, grad_alpha, grad_base) and of grad_x over all tokens,
against which the HIP kernels' fp32 accumulation is held to tight bounds.
"""

from __future__ import annotations

import numpy as np
import torch

from oracle import mhc_oracle as orc


def close_gpu(got, want, rtol, atol, what="", chunk=4096):
    """torch.allclose semantics (|got - want| <= atol + rtol |want|) evaluated
    on the device in float64, chunked over the first dimension; reports the
    number of elements outside the bound and the largest error."""
    assert tuple(got.shape) == tuple(want.shape), (what, tuple(got.shape), tuple(want.shape))
    got, want = got.detach(), want.detach()
    g = got.reshape(got.shape[0], -1) if got.dim() > 1 else got.reshape(-1, 1)
    w = want.reshape(want.shape[0], -1) if want.dim() > 1 else want.reshape(-1, 1)
    bad, worst = 0, 0.0
    for s in range(0, g.shape[0], chunk):
        a = g[s:s + chunk].double()
        b = w[s:s + chunk].to(a.device).double()
        err = (a - b).abs()
        bad += int((err > atol + rtol * b.abs()).sum())
        worst = max(worst, float(err.max()) if err.numel() else 0.0)
    assert bad == 0, f"{what}: {bad} / {g.numel()} outside tol, max err {worst:.3e}"
    return worst


def pre_bwd_fp64(x, phi, alpha, base, grad_y, grad_post_out, grad_comb_frag, kw,
                 grad_x=None, chunk=2048):
    """Float64 VJP of mhc_pre_clamp_sinkhorn over all tokens (the oracle's
    pre_bwd, with its contractions on the device).

    Returns a dict with grad_phi (device, float64), grad_alpha and grad_base
    (numpy float64).  When ``grad_x`` (the kernel's output) is given, it is
    compared chunk by chunk with the float64 grad_x at the bf16 tolerance
    (rtol / atol 2e-2), and the largest error is returned as "grad_x_err"."""
    T, N, D = x.shape
    M, K = 2 * N + N * N, N * D
    dev = x.device
    norm_eps = kw.get("norm_eps", 1e-6)
    hc_eps = kw.get("hc_eps", 1e-6)
    phi64 = phi.double().reshape(M, K)
    inv = torch.empty(T, dtype=torch.float64, device=dev)
    mixes = torch.empty(T, M, dtype=torch.float64, device=dev)
    grad_pre = torch.empty(T, N, dtype=torch.float64, device=dev)
    gy = grad_y.reshape(T, D)
    for s in range(0, T, chunk):
        xc = x[s:s + chunk].double().reshape(-1, K)
        ic = 1.0 / torch.sqrt((xc * xc).mean(dim=-1) + norm_eps)
        inv[s:s + chunk] = ic
        mixes[s:s + chunk] = (xc * ic[:, None]) @ phi64.t()
        grad_pre[s:s + chunk] = (xc.view(-1, N, D) * gy[s:s + chunk].double().view(-1, 1, D)).sum(-1)
        del xc
    host = lambda t: t.detach().double().cpu().numpy()
    gm, ga, gb = orc.small_stage_bwd(
        host(mixes), host(grad_pre), host(grad_post_out), host(grad_comb_frag), host(alpha),
        host(base), N, hc_eps=hc_eps, clamp_min=kw.get("clamp_min", 0.0),
        clamp_max=kw.get("clamp_max", 0.0), iter_times=kw.get("iter_times", 20))
    gm = torch.from_numpy(gm).to(dev)
    g = gm * inv[:, None]                      # grad_phi = sum_t gm_t (x)_t * inv_t
    grad_phi = torch.zeros(M, K, dtype=torch.float64, device=dev)
    a64 = alpha.double().to(dev)
    pre = torch.sigmoid(mixes[:, :N] * a64[0] + base.double().to(dev)[:N]) + hc_eps
    gx_err = None
    for s in range(0, T, chunk):
        xc = x[s:s + chunk].double().reshape(-1, K)
        grad_phi += g[s:s + chunk].t() @ xc
        if grad_x is not None:
            gs = gm[s:s + chunk] @ phi64
            ic = inv[s:s + chunk]
            dot = (xc * gs).sum(-1)
            gx = ic[:, None] * gs - (ic ** 3 * dot / K)[:, None] * xc
            gx = gx.view(-1, N, D) + gy[s:s + chunk].double().view(-1, 1, D) * pre[s:s + chunk, :, None]
            e = close_gpu(grad_x[s:s + chunk], gx, 2e-2, 2e-2, f"grad_x tokens {s}..")
            gx_err = e if gx_err is None else max(gx_err, e)
        del xc
    return {"grad_phi": grad_phi, "grad_alpha": ga, "grad_base": gb, "grad_x_err": gx_err,
            "mixes": mixes, "inv_rms": inv}


def check_reductions(got_phi, got_alpha, got_base, ref, what="", rtol=1e-4, atol_frac=1e-5):
    """The pre backward's T-reductions against a float64 reference: rtol 1e-4
    with atol 1e-5 * max|ref| (the fp32 fixed-order sums measure a few 1e-6 of
    max|grad_phi| against float64 at up to 65536 tokens)."""
    rp = ref["grad_phi"]
    close_gpu(got_phi.reshape(rp.shape), rp, rtol, atol_frac * float(rp.abs().max()), what + " grad_phi")
    for got, w, name in ((got_alpha, ref["grad_alpha"], "grad_alpha"),
                         (got_base, ref["grad_base"], "grad_base")):
        w = torch.from_numpy(np.asarray(w)).to(got.device)
        close_gpu(got, w, rtol, atol_frac * float(w.abs().max()), what + " " + name)
