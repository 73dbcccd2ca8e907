"""The package's public ``*_ref`` functions (pure PyTorch, part of the drop-in
API) against the oracle, on CPU.  The pre backward comparison sets torch
autograd (through ``mhc_pre_clamp_sinkhorn_backward_ref``) against the
oracle's hand-written VJP: two independent derivations."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from FlagOS_mhc import (
    mhc_post_backward_ref,
    mhc_post_ref,
    mhc_pre_clamp_sinkhorn_backward_ref,
    mhc_pre_clamp_sinkhorn_ref,
)
from oracle import mhc_oracle as orc


def _t(a, dtype=torch.float32):
    return torch.tensor(np.asarray(a), dtype=torch.float64).to(dtype)


def _close(got, want, rtol, atol):
    got = got.detach().double().numpy() if isinstance(got, torch.Tensor) else got
    np.testing.assert_allclose(got, want, rtol=rtol, atol=atol)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape4", [True, False])
def test_post_ref_vs_oracle(rng, dtype, shape4):
    B, S, N, D = 2, 8, 4, 64
    x = _t(rng.standard_normal((B * S, N, D)), dtype)
    h_res = _t(rng.standard_normal((B * S, N, N)))
    h_out = _t(rng.standard_normal((B * S, D)), dtype)
    h_post = _t(rng.standard_normal((B * S, N)))
    want = orc.post_fwd(x.double(), h_res.double(), h_out.double(), h_post.double())
    args = (x, h_res, h_out, h_post)
    if shape4:
        args = (x.reshape(B, S, N, D), h_res.reshape(B, S, N, N), h_out.reshape(B, S, D),
                h_post.reshape(B, S, N))
    y = mhc_post_ref(*args)
    assert y.dtype == dtype and y.shape == args[0].shape
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    _close(y.reshape(B * S, N, D), want, tol, tol)


@pytest.mark.parametrize("N", [4, 8])
def test_post_bwd_ref_vs_oracle(rng, N):
    T, D = 16, 32
    x = _t(rng.standard_normal((T, N, D)), torch.bfloat16)
    h_res = _t(rng.standard_normal((T, N, N)))
    h_out = _t(rng.standard_normal((T, D)), torch.bfloat16)
    h_post = _t(rng.standard_normal((T, N)))
    gy = _t(rng.standard_normal((T, N, D)), torch.bfloat16)
    got = mhc_post_backward_ref(gy, x, h_res, h_out, h_post)
    want = orc.post_bwd(gy.double(), x.double(), h_res.double(), h_out.double(), h_post.double())
    assert got[0].dtype == torch.bfloat16 and got[1].dtype == torch.float32
    for g, w, tol in zip(got, want, (1e-2, 1e-5, 1e-2, 1e-5)):
        _close(g, w, tol, tol)


def _pre_case(rng, T, N, D, phi_dtype=torch.float32, x_scale=0.1):
    M = 2 * N + N * N
    x = _t(rng.standard_normal((T, N, D)) * x_scale, torch.bfloat16)
    phi = _t(rng.standard_normal((M, N * D)) * 0.1, phi_dtype)
    alpha = _t([0.5, 0.5, 0.5])
    base = _t(rng.standard_normal(M) * 0.01)
    return x, phi, alpha, base


# the reference's own test case (tests/test_correctness.py:72-115): B,S,N,D = 2,8,4,64
@pytest.mark.parametrize("N,clamp,iters", [(4, 3.0, 20), (4, 0.0, 20), (8, 3.0, 20), (4, 3.0, 1)])
def test_pre_ref_vs_oracle(rng, N, clamp, iters):
    T, D = 16, 64
    x, phi, alpha, base = _pre_case(rng, T, N, D)
    kw = dict(norm_eps=1e-6, hc_eps=1e-6, clamp_min=-clamp, clamp_max=clamp, iter_times=iters)
    got = mhc_pre_clamp_sinkhorn_ref(x.reshape(2, 8, N, D), phi, alpha, base, **kw)
    want = orc.pre_fwd(x.double(), phi.double(), alpha.double(), base.double(), **kw)
    assert got["y"].shape == (2, 8, D) and got["y"].dtype == torch.bfloat16
    _close(got["y"].reshape(T, D), want["y"], 1e-2, 1e-2)
    for k in ("post_out", "comb_frag", "inv_rms", "mixes", "h_res_logits", "pre"):
        _close(got[k], want[k], 1e-4, 1e-5)


@pytest.mark.parametrize("N,clamp,iters", [(4, 3.0, 20), (4, 0.0, 5), (8, 0.5, 20), (4, 0.3, 40)])
def test_pre_bwd_ref_autograd_vs_oracle_vjp(rng, N, clamp, iters):
    T, D = 16, 64
    x, phi, alpha, base = _pre_case(rng, T, N, D, x_scale=1.0)
    gy = _t(rng.standard_normal((T, D)), torch.bfloat16)
    gpost = _t(rng.standard_normal((T, N)))
    gcomb = _t(rng.standard_normal((T, N, N)))
    kw = dict(norm_eps=1e-6, hc_eps=1e-6, clamp_min=-clamp, clamp_max=clamp, iter_times=iters)
    got = mhc_pre_clamp_sinkhorn_backward_ref(x, phi, alpha, base, gy, gpost, gcomb, **kw)
    want = orc.pre_bwd(x.double(), phi.double(), alpha.double(), base.double(), gy.double(),
                       gpost.double(), gcomb.double(), **kw)
    assert got[0].dtype == torch.bfloat16
    _close(got[0], want[0], 2e-2, 2e-2)
    for g, w in zip(got[1:], want[1:]):
        scale = np.abs(w).max()
        _close(g, w, 1e-3, 1e-4 * scale)


def clamp_bound_base(N, c, rng):
    """base for phi = 0: mixes are then exactly 0 and the logits equal
    base[2N:] bit for bit, so entries can sit exactly on a clamp bound.  Row i
    of the N x N logits holds +c, -c, a value inside and a value outside the
    range (the rest random inside)."""
    M = 2 * N + N * N
    base = rng.uniform(-0.5, 0.5, M) * c
    lg = base[2 * N:].reshape(N, N)
    for i in range(N):
        lg[i, i % N] = c
        lg[i, (i + 1) % N] = -c
        lg[i, (i + 2) % N] = 1.5 * c * (1 if i % 2 else -1)
    base[2 * N:] = lg.reshape(-1)
    return base.astype(np.float32)


@pytest.mark.parametrize("N", [4, 8])
def test_clamp_gradient_inclusive_at_bounds(rng, N):
    """F7: the reference's *_ref passes the clamp gradient where the logit
    equals a bound (torch.clamp autograd, src/mhc_pre_clamp_sinkhorn_backward.py:
    1434-1435); its Triton kernel masks them out (strict, :1186-1191).  With
    phi = 0 the logits are exactly base, some exactly on +-clamp: the oracle's
    grad_base must match torch autograd through the package's *_ref there, and
    a strict mask (the Triton semantics, planted here in a copy of the oracle's
    result) must not."""
    T, D, c = 8, 32, 0.5
    M = 2 * N + N * N
    x = _t(rng.standard_normal((T, N, D)))
    phi = torch.zeros(M, N * D)
    alpha = torch.tensor([0.5, 0.5, 1.0])
    base = torch.from_numpy(clamp_bound_base(N, c, rng))
    gy = _t(rng.standard_normal((T, D)))
    gpost = _t(rng.standard_normal((T, N)))
    gcomb = _t(rng.standard_normal((T, N, N)))
    kw = dict(norm_eps=1e-6, hc_eps=1e-6, clamp_min=-c, clamp_max=c, iter_times=20)
    logits = orc.pre_fwd(x.double(), phi.double(), alpha.double(), base.double(), **kw)["h_res_logits"]
    lg = base.double().numpy()[2 * N:].reshape(N, N)
    assert np.array_equal(logits, np.broadcast_to(lg, (T, N, N)))   # logits == base exactly
    on_bound = np.abs(lg) == c
    outside = np.abs(lg) > c
    assert on_bound.sum() == 2 * N and outside.sum() == N

    got = mhc_pre_clamp_sinkhorn_backward_ref(x, phi, alpha, base, gy, gpost, gcomb, **kw)
    want = orc.pre_bwd(x.double(), phi.double(), alpha.double(), base.double(), gy.double(),
                       gpost.double(), gcomb.double(), **kw)
    gb_torch, gb_orc = got[3].double().numpy(), want[3]
    scale = np.abs(gb_orc).max()
    np.testing.assert_allclose(gb_torch, gb_orc, rtol=1e-4, atol=1e-5 * scale)
    gl = gb_orc[2 * N:].reshape(N, N)
    scale_l = np.abs(gl).max()
    np.testing.assert_allclose(gb_torch[2 * N:].reshape(N, N), gl, rtol=1e-4, atol=1e-5 * scale_l)
    assert (gl[on_bound] != 0).all()                         # gradient passes at the bounds
    assert (gl[outside] == 0).all()                          # and not outside them
    strict = gl * ~on_bound                                   # Triton's strict mask
    assert not np.allclose(strict, gb_torch[2 * N:].reshape(N, N), rtol=1e-4, atol=1e-5 * scale_l)
