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
