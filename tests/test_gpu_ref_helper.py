"""CPU checks of the full-size float64 reference used by the GPU parity tests
(tests/gpu_ref.py): on small shapes it must reproduce the oracle's pre_bwd
exactly (same float64 formulas, contractions done by torch instead of numpy),
and its comparison helper must flag a planted error."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from gpu_ref import check_reductions, close_gpu, pre_bwd_fp64
from oracle import mhc_oracle as orc


@pytest.mark.parametrize("N,T,D,clamp,iters", [(4, 37, 24, 0.5, 20), (8, 9, 16, 3.0, 7), (4, 5, 8, 0.0, 1)])
def test_pre_bwd_fp64_matches_oracle(rng, N, T, D, clamp, iters):
    M = 2 * N + N * N
    x = torch.from_numpy(rng.standard_normal((T, N, D)))
    phi = torch.from_numpy(rng.standard_normal((M, N * D)) * 0.3)
    alpha = torch.tensor([0.5, 0.7, 1.1], dtype=torch.float64)
    base = torch.from_numpy(rng.standard_normal(M) * 0.1)
    gy = torch.from_numpy(rng.standard_normal((T, D)))
    gpost = torch.from_numpy(rng.standard_normal((T, N)))
    gcomb = torch.from_numpy(rng.standard_normal((T, N, N)))
    kw = dict(norm_eps=1e-6, hc_eps=1e-6, clamp_min=-clamp, clamp_max=clamp, iter_times=iters)
    want = orc.pre_bwd(x.numpy(), phi.numpy(), alpha.numpy(), base.numpy(), gy.numpy(),
                       gpost.numpy(), gcomb.numpy(), **kw)
    got = pre_bwd_fp64(x, phi, alpha, base, gy, gpost, gcomb, kw,
                       grad_x=torch.from_numpy(want[0]), chunk=4)
    np.testing.assert_allclose(got["grad_phi"].numpy(), want[1], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(got["grad_alpha"], want[2], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(got["grad_base"], want[3], rtol=1e-12, atol=1e-12)
    assert got["grad_x_err"] < 1e-10
    check_reductions(torch.from_numpy(want[1]), torch.from_numpy(want[2]),
                     torch.from_numpy(want[3]), got)
    # a planted error of 3e-5 * max in one grad_phi element must fail the bound
    bad = torch.from_numpy(want[1].copy())
    bad[1, 2] += 3e-5 * float(np.abs(want[1]).max()) + 2e-4 * abs(float(bad[1, 2]))
    with pytest.raises(AssertionError):
        check_reductions(bad, torch.from_numpy(want[2]), torch.from_numpy(want[3]), got)


def test_close_gpu_counts_outliers():
    a = torch.zeros(10, 3)
    b = torch.zeros(10, 3)
    b[7, 1] = 1.0
    close_gpu(a, a, 0.0, 0.0, chunk=3)
    with pytest.raises(AssertionError, match="1 / 30"):
        close_gpu(a, b, 1e-3, 1e-3, chunk=3)
