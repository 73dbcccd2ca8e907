"""CPU oracle for the four mHC operators.  TEST INFRASTRUCTURE ONLY.

This module is the checker, never the product: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it.  The shipped operators (package ``FlagOS_mhc``) never call it and
fail loudly when their HIP library is missing.

It restates, in float64 numpy and independently of torch, the semantics of the
reference's PyTorch ``*_ref`` functions (the reference's parity contract):

* ``post_fwd``  -- ``src/mhc_post.py:344-352``  (mhc_post_ref)
* ``post_bwd``  -- ``src/mhc_post_backward.py:624-643`` (mhc_post_backward_ref)
* ``pre_fwd``   -- ``src/mhc_pre_clamp_sinkhorn.py:974-1022``
                   (mhc_pre_clamp_sinkhorn_ref)
* ``pre_bwd``   -- ``src/mhc_pre_clamp_sinkhorn_backward.py:1397-1453``
                   (mhc_pre_clamp_sinkhorn_backward_ref).  The reference gets
                   this one from torch autograd; here every vector-Jacobian
                   product is written out by hand (Sinkhorn row/column
                   normalisation, softmax, clamp, sigmoid heads, RMSNorm), so
                   that autograd and this file are two independent derivations.

All arithmetic is float64 on float64 copies of the inputs; the caller casts
outputs to whatever storage dtype it compares against.

How each function is pinned (tests/test_oracle.py):

* post_fwd: brute-force Python loops on tiny shapes, h_res = I / h_post = 0
  gives y = x, permutation h_res permutes streams, linearity in (x, h_out).
* post_bwd: central finite differences of <gy, post_fwd(...)> along random
  directions (exact for a bilinear map), the adjoint (dot-product) identity.
* pre_fwd: RMS of a constant row, mixes against a brute-force loop, the
  sigmoid identity at zero, Sinkhorn on constant logits against its scalar
  recurrence, iter_times = 1 against softmax + one column normalisation written
  element by element, the doubly-stochastic invariant, clamp saturation.
* pre_bwd: central finite differences of the scalar loss
  <gy, y> + <gpost, post_out> + <gcomb, comb_frag> with respect to x, phi,
  alpha and base, and agreement with torch.autograd through an independent
  torch restatement (the package's public ``*_ref`` functions).

Golden vectors: the reference ships none (its only test compares two live
computations, ``tests/test_correctness.py:25-32``); the fixtures under
``tests/golden/`` are written by this oracle and pin regressions only.
"""

from __future__ import annotations

import numpy as np

__all__ = [
    "post_fwd",
    "post_bwd",
    "pre_fwd",
    "pre_bwd",
    "sinkhorn_fwd",
    "sinkhorn_bwd",
    "small_stage_bwd",
]


def _f64(a):
    return np.asarray(a, dtype=np.float64)


# ---------------------------------------------------------------------------
# mhc_post
# ---------------------------------------------------------------------------
def post_fwd(x, h_res, h_out, h_post):
    """y[t,i,:] = sum_j h_res[t,j,i] * x[t,j,:] + h_post[t,i] * h_out[t,:].

    Follows ``src/mhc_post.py:344-352``: note the transposed use of h_res
    (column i of the per-token N x N matrix feeds output stream i).
    Shapes: x (T,N,D), h_res (T,N,N), h_out (T,D), h_post (T,N) -> (T,N,D).
    """
    x, h_res, h_out, h_post = map(_f64, (x, h_res, h_out, h_post))
    T, N, D = x.shape
    y = np.matmul(np.swapaxes(h_res, 1, 2), x)          # (T,N,N)^T @ (T,N,D)
    y += h_post[:, :, None] * h_out[:, None, :]
    return y


def post_bwd(grad_y, x, h_res, h_out, h_post):
    """VJPs of post_fwd; follows ``src/mhc_post_backward.py:624-643``.

    Returns (grad_x (T,N,D), grad_h_res (T,N,N), grad_h_out (T,D),
    grad_h_post (T,N)).
    """
    gy, x, h_res, h_out, h_post = map(_f64, (grad_y, x, h_res, h_out, h_post))
    grad_x = np.matmul(h_res, gy)                          # sum_i h_res[j,i] gy[i]
    grad_h_res = np.matmul(x, np.swapaxes(gy, 1, 2))      # [j,i] = <x[j], gy[i]>
    grad_h_out = np.einsum("ti,tid->td", h_post, gy)
    grad_h_post = np.einsum("td,tid->ti", h_out, gy)
    return grad_x, grad_h_res, grad_h_out, grad_h_post


# ---------------------------------------------------------------------------
# Sinkhorn stage (per token N x N)
# ---------------------------------------------------------------------------
def _softmax_rows(z):
    z = z - z.max(axis=-1, keepdims=True)
    e = np.exp(z)
    return e / e.sum(axis=-1, keepdims=True)


def sinkhorn_fwd(logits_c, hc_eps, iter_times, keep_states=False):
    """Row-softmax, + hc_eps, one column normalisation, then
    ``iter_times - 1`` (row, column) normalisation pairs, every denominator
    being ``sum + hc_eps``.

    Follows ``src/mhc_pre_clamp_sinkhorn.py:1004-1010`` exactly, including the
    placement of hc_eps: added to the softmax output *after* the division.
    ``iter_times <= 1`` leaves only the first column normalisation (the
    reference loops over ``range(iter_times - 1)``).
    """
    s = _softmax_rows(logits_c)
    m0 = s + hc_eps
    ic0 = 1.0 / (m0.sum(axis=-2, keepdims=True) + hc_eps)
    c = m0 * ic0
    states = []
    for _ in range(max(int(iter_times) - 1, 0)):
        ir = 1.0 / (c.sum(axis=-1, keepdims=True) + hc_eps)
        r = c * ir
        ic = 1.0 / (r.sum(axis=-2, keepdims=True) + hc_eps)
        c_new = r * ic
        if keep_states:
            states.append((r, ir, c_new, ic))
        c = c_new
    if keep_states:
        return c, (s, m0, ic0, states)
    return c


def sinkhorn_bwd(grad_c, saved):
    """Hand-derived VJP of :func:`sinkhorn_fwd` with respect to the clamped
    logits.

    Column normalisation ``out = u * ic`` with ``ic = 1/(colsum(u)+eps)`` has
    VJP ``du = ic * (g - colsum(g * out))``; the row normalisation is the same
    along rows; softmax has ``dz = s * (g - rowsum(g * s))``.  The reference
    obtains the same quantity from torch autograd
    (``src/mhc_pre_clamp_sinkhorn_backward.py:1440-1453``); its hand-written
    Triton walk (``:1120-1163``) uses these formulas too.
    """
    s, m0, ic0, states = saved
    g = grad_c
    for (r, ir, c_new, ic) in reversed(states):
        g = ic * (g - (g * c_new).sum(axis=-2, keepdims=True))   # through column norm
        g = ir * (g - (g * r).sum(axis=-1, keepdims=True))       # through row norm
    c0 = m0 * ic0
    g = ic0 * (g - (g * c0).sum(axis=-2, keepdims=True))         # first column norm
    # m0 = s + eps: identity; softmax VJP
    return s * (g - (g * s).sum(axis=-1, keepdims=True))


# ---------------------------------------------------------------------------
# mhc_pre_clamp_sinkhorn
# ---------------------------------------------------------------------------
def _sigmoid(z):
    return 1.0 / (1.0 + np.exp(-z))


def _clamp_enabled(clamp_min, clamp_max):
    # src/mhc_pre_clamp_sinkhorn.py:1000 -- enabled iff either bound is non-zero
    return clamp_min != 0.0 or clamp_max != 0.0


def pre_fwd(x, phi, alpha, base, norm_eps=1e-6, hc_eps=1e-6,
            clamp_min=0.0, clamp_max=0.0, iter_times=20):
    """Forward of mhc_pre_clamp_sinkhorn, ``src/mhc_pre_clamp_sinkhorn.py:974-1022``.

    x (T,N,D); phi (M, N*D) with M = 2N + N^2; alpha (3,); base (M,).
    Returns a dict with y (T,D), post_out (T,N), comb_frag (T,N,N), inv_rms
    (T,), mixes (T,M), h_res_logits (T,N,N) (pre-clamp), pre (T,N),
    x_scaled (T,N*D).
    """
    x, phi, alpha, base = map(_f64, (x, phi, alpha, base))
    T, N, D = x.shape
    xf = x.reshape(T, N * D)
    inv = 1.0 / np.sqrt((xf * xf).mean(axis=-1) + norm_eps)
    x_scaled = xf * inv[:, None]
    mixes = x_scaled @ phi.T
    pre = _sigmoid(mixes[:, :N] * alpha[0] + base[:N]) + hc_eps
    post = 2.0 * _sigmoid(mixes[:, N:2 * N] * alpha[1] + base[N:2 * N])
    logits = (mixes[:, 2 * N:] * alpha[2] + base[2 * N:]).reshape(T, N, N)
    lc = np.clip(logits, clamp_min, clamp_max) if _clamp_enabled(clamp_min, clamp_max) else logits
    comb = sinkhorn_fwd(lc, hc_eps, iter_times)
    y = (x * pre[:, :, None]).sum(axis=1)
    return {
        "y": y,
        "post_out": post,
        "comb_frag": comb,
        "inv_rms": inv,
        "mixes": mixes,
        "h_res_logits": logits,
        "pre": pre,
        "x_scaled": x_scaled,
    }


def small_stage_bwd(mixes, grad_pre, grad_post_out, grad_comb_frag, alpha, base, N,
                    hc_eps=1e-6, clamp_min=0.0, clamp_max=0.0, iter_times=20):
    """VJP of the per-token heads, clamp, softmax and Sinkhorn of
    :func:`pre_fwd` with respect to mixes, alpha and base, given
    grad_pre = d loss / d pre (T,N) (the reference's ``_small_stage_bwd``,
    ``src/mhc_pre_clamp_sinkhorn_backward.py:1251-1286``, semantics of the
    autograd path ``:1428-1453``).

    Returns (grad_mixes (T,M), grad_alpha (3,), grad_base (M,)).  The clamp
    gradient passes where ``clamp_min <= logit <= clamp_max`` (inclusive, as
    torch.clamp's backward; ``:1434-1435``).
    """
    mixes, grad_pre, alpha, base = map(_f64, (mixes, grad_pre, alpha, base))
    T = mixes.shape[0]
    gpost = _f64(grad_post_out).reshape(T, N)
    gcomb = _f64(grad_comb_frag).reshape(T, N, N)
    z_pre = mixes[:, :N] * alpha[0] + base[:N]
    z_post = mixes[:, N:2 * N] * alpha[1] + base[N:2 * N]
    ml = mixes[:, 2 * N:].reshape(T, N, N)
    logits = ml * alpha[2] + base[2 * N:].reshape(N, N)
    clamp = _clamp_enabled(clamp_min, clamp_max)
    lc = np.clip(logits, clamp_min, clamp_max) if clamp else logits
    _, saved = sinkhorn_fwd(lc, hc_eps, iter_times, keep_states=True)
    sp = _sigmoid(z_pre)
    spo = _sigmoid(z_post)
    dz_pre = grad_pre * sp * (1.0 - sp)
    dz_post = gpost * 2.0 * spo * (1.0 - spo)
    dlc = sinkhorn_bwd(gcomb, saved)
    if clamp:
        dlc = dlc * ((logits >= clamp_min) & (logits <= clamp_max))
    grad_mixes = np.concatenate(
        [dz_pre * alpha[0], dz_post * alpha[1], (dlc * alpha[2]).reshape(T, N * N)], axis=1)
    grad_alpha = np.array([
        (dz_pre * mixes[:, :N]).sum(),
        (dz_post * mixes[:, N:2 * N]).sum(),
        (dlc * ml).sum(),
    ])
    grad_base = np.concatenate(
        [dz_pre.sum(axis=0), dz_post.sum(axis=0), dlc.sum(axis=0).reshape(N * N)])
    return grad_mixes, grad_alpha, grad_base


def pre_bwd(x, phi, alpha, base, grad_y, grad_post_out, grad_comb_frag,
            norm_eps=1e-6, hc_eps=1e-6, clamp_min=0.0, clamp_max=0.0,
            iter_times=20, return_intermediates=False):
    """Hand-derived VJP of :func:`pre_fwd` for the loss
    ``<grad_y, y> + <grad_post_out, post_out> + <grad_comb_frag, comb_frag>``
    (``src/mhc_pre_clamp_sinkhorn_backward.py:1440-1453``).

    Returns (grad_x (T,N,D), grad_phi (M,N*D), grad_alpha (3,), grad_base (M,)).
    Clamp gradient passes where ``clamp_min <= logit <= clamp_max``
    (inclusive, as torch.clamp's backward; ``:1434-1435``).
    """
    x, phi, alpha, base = map(_f64, (x, phi, alpha, base))
    gy, gpost, gcomb = map(_f64, (grad_y, grad_post_out, grad_comb_frag))
    T, N, D = x.shape
    M = 2 * N + N * N
    xf = x.reshape(T, N * D)
    gy = gy.reshape(T, D)
    gpost = gpost.reshape(T, N)
    gcomb = gcomb.reshape(T, N, N)

    # --- forward recompute -------------------------------------------------
    inv = 1.0 / np.sqrt((xf * xf).mean(axis=-1) + norm_eps)
    x_scaled = xf * inv[:, None]
    mixes = x_scaled @ phi.T
    pre = _sigmoid(mixes[:, :N] * alpha[0] + base[:N]) + hc_eps

    # --- small stage -------------------------------------------------------
    grad_pre = np.einsum("td,tnd->tn", gy, x)             # from y = sum_n x[n] pre[n]
    grad_mixes, grad_alpha, grad_base = small_stage_bwd(
        mixes, grad_pre, gpost, gcomb, alpha, base, N, hc_eps=hc_eps, clamp_min=clamp_min,
        clamp_max=clamp_max, iter_times=iter_times)

    # --- contraction and RMSNorm backward ---------------------------------
    gs = grad_mixes @ phi                                  # d loss / d x_scaled
    grad_phi = grad_mixes.T @ x_scaled
    dot = (xf * gs).sum(axis=-1)
    # x_scaled = x * inv, inv = (mean(x^2)+eps)^-1/2  =>  d inv/dx = -inv^3 x / ND
    grad_xf = inv[:, None] * gs - (inv ** 3 * dot / (N * D))[:, None] * xf
    grad_x = grad_xf.reshape(T, N, D) + gy[:, None, :] * pre[:, :, None]
    assert grad_mixes.shape == (T, M)
    if return_intermediates:
        return grad_x, grad_phi, grad_alpha, grad_base, {
            "grad_pre": grad_pre, "grad_mixes": grad_mixes, "inv_rms": inv, "mixes": mixes}
    return grad_x, grad_phi, grad_alpha, grad_base
