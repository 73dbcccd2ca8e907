"""Pins the CPU oracle (oracle/mhc_oracle.py) against checks that do not
restate its formulas: brute-force loops, closed forms, invariants and central
finite differences of its own forward.  CPU only."""

from __future__ import annotations

import itertools

import numpy as np
import pytest

from oracle import mhc_oracle as orc


def _sig(z):
    return 1.0 / (1.0 + np.exp(-z))


# ---------------------------------------------------------------------------
# mhc_post forward
# ---------------------------------------------------------------------------
def _post_inputs(rng, T, N, D):
    return (rng.standard_normal((T, N, D)), rng.standard_normal((T, N, N)),
            rng.standard_normal((T, D)), rng.standard_normal((T, N)))


@pytest.mark.parametrize("N", [2, 4, 8])
def test_post_fwd_brute_force(rng, N):
    T, D = 3, 5
    x, hr, ho, hp = _post_inputs(rng, T, N, D)
    y = orc.post_fwd(x, hr, ho, hp)
    for t, i, d in itertools.product(range(T), range(N), range(D)):
        want = hp[t, i] * ho[t, d]
        for j in range(N):
            want += hr[t, j, i] * x[t, j, d]
        assert abs(y[t, i, d] - want) < 1e-12


def test_post_fwd_identity_and_permutation(rng):
    T, N, D = 4, 4, 16
    x, _, ho, _ = _post_inputs(rng, T, N, D)
    eye = np.broadcast_to(np.eye(N), (T, N, N))
    np.testing.assert_array_equal(orc.post_fwd(x, eye, ho, np.zeros((T, N))), x)
    perm = [2, 0, 3, 1]                      # stream j feeds output stream perm[j]
    P = np.zeros((T, N, N))
    for j, i in enumerate(perm):
        P[:, j, i] = 1.0
    y = orc.post_fwd(x, P, ho, np.zeros((T, N)))
    for j, i in enumerate(perm):
        np.testing.assert_array_equal(y[:, i], x[:, j])
    # h_res = 0, h_post = e_1: only stream 1 receives h_out
    hp = np.zeros((T, N))
    hp[:, 1] = 1.0
    y = orc.post_fwd(x, np.zeros((T, N, N)), ho, hp)
    np.testing.assert_array_equal(y[:, 1], ho)
    assert not y[:, [0, 2, 3]].any()


# ---------------------------------------------------------------------------
# mhc_post backward: finite differences of <gy, post_fwd>
# ---------------------------------------------------------------------------
def _fd(f, args, idx, v, eps=1e-6):
    a_p = list(args)
    a_m = list(args)
    a_p[idx] = args[idx] + eps * v
    a_m[idx] = args[idx] - eps * v
    return (f(*a_p) - f(*a_m)) / (2 * eps)


@pytest.mark.parametrize("N", [2, 4, 8])
def test_post_bwd_finite_differences(rng, N):
    T, D = 3, 7
    args = _post_inputs(rng, T, N, D)
    gy = rng.standard_normal((T, N, D))
    loss = lambda *a: float((gy * orc.post_fwd(*a)).sum())
    grads = orc.post_bwd(gy, *args)
    for idx in range(4):
        v = rng.standard_normal(args[idx].shape)
        want = _fd(loss, args, idx, v)
        got = float((grads[idx] * v).sum())
        assert abs(got - want) <= 1e-7 * (1 + abs(want)), (idx, got, want)


def test_post_bwd_brute_force(rng):
    T, N, D = 2, 4, 3
    x, hr, ho, hp = _post_inputs(rng, T, N, D)
    gy = rng.standard_normal((T, N, D))
    gx, ghr, gho, ghp = orc.post_bwd(gy, x, hr, ho, hp)
    for t in range(T):
        for j, i in itertools.product(range(N), range(N)):
            assert abs(ghr[t, j, i] - sum(x[t, j, d] * gy[t, i, d] for d in range(D))) < 1e-12
        for i in range(N):
            assert abs(ghp[t, i] - sum(ho[t, d] * gy[t, i, d] for d in range(D))) < 1e-12
        for d in range(D):
            assert abs(gho[t, d] - sum(hp[t, i] * gy[t, i, d] for i in range(N))) < 1e-12
            for j in range(N):
                assert abs(gx[t, j, d] - sum(hr[t, j, i] * gy[t, i, d] for i in range(N))) < 1e-12


# ---------------------------------------------------------------------------
# Sinkhorn stage
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("N,iters", [(4, 1), (4, 20), (8, 20), (8, 3)])
def test_sinkhorn_constant_logits_recurrence(N, iters):
    eps = 1e-3  # large, so a misplaced eps shows up
    lc = np.full((2, N, N), 0.7)
    c = orc.sinkhorn_fwd(lc, eps, iters)
    a = 1.0 / N + eps                     # softmax of a constant row, + eps
    a = a / (N * a + eps)                 # first column normalisation
    for _ in range(iters - 1):
        a = a / (N * a + eps)             # row
        a = a / (N * a + eps)             # column
    np.testing.assert_allclose(c, a, rtol=1e-14, atol=0)


def test_sinkhorn_single_iteration_elementwise(rng):
    N, eps = 4, 1e-2
    lc = rng.standard_normal((N, N)) * 2
    c = orc.sinkhorn_fwd(lc[None], eps, 1)[0]
    s = np.empty((N, N))
    for i in range(N):
        row = [np.exp(lc[i, j]) for j in range(N)]
        for j in range(N):
            s[i, j] = row[j] / sum(row) + eps
    for i, j in itertools.product(range(N), range(N)):
        want = s[i, j] / (sum(s[k, j] for k in range(N)) + eps)
        assert abs(c[i, j] - want) < 1e-14
    # iter_times = 0 behaves like 1 (the reference loops over range(iters - 1))
    np.testing.assert_array_equal(orc.sinkhorn_fwd(lc[None], eps, 0), c[None])


@pytest.mark.parametrize("N", [4, 8])
def test_sinkhorn_doubly_stochastic(rng, N):
    lc = rng.standard_normal((5, N, N)) * 3
    c = orc.sinkhorn_fwd(lc, 0.0, 300)
    np.testing.assert_allclose(c.sum(axis=-2), 1.0, atol=1e-13)
    np.testing.assert_allclose(c.sum(axis=-1), 1.0, atol=1e-9)
    # with eps > 0 every column sum is S / (S + eps) < 1
    c = orc.sinkhorn_fwd(lc, 1e-6, 20)
    cs = c.sum(axis=-2)
    assert np.all(cs < 1.0) and np.all(cs > 1.0 - 1e-5)


def test_sinkhorn_permutation_equivariance(rng):
    N = 4
    lc = rng.standard_normal((N, N))
    pr, pc = [3, 1, 0, 2], [1, 2, 3, 0]
    c = orc.sinkhorn_fwd(lc[None], 1e-6, 20)[0]
    cp = orc.sinkhorn_fwd(lc[pr][:, pc][None], 1e-6, 20)[0]
    np.testing.assert_allclose(cp, c[pr][:, pc], rtol=1e-13)


# ---------------------------------------------------------------------------
# pre forward
# ---------------------------------------------------------------------------
def _pre_inputs(rng, T, N, D, phi_scale=None):
    M = 2 * N + N * N
    x = rng.standard_normal((T, N, D))
    phi = rng.standard_normal((M, N * D)) * (phi_scale or 1.0 / np.sqrt(N * D))
    alpha = np.array([0.5, 0.7, 1.3])
    base = rng.standard_normal(M) * 0.1
    return x, phi, alpha, base


def test_pre_rms_constant_rows():
    T, N, D = 3, 4, 8
    c = np.array([0.5, 2.0, 1e-4])
    x = np.broadcast_to(c[:, None, None], (T, N, D)).copy()
    M = 2 * N + N * N
    out = orc.pre_fwd(x, np.zeros((M, N * D)), np.ones(3), np.zeros(M), norm_eps=1e-6)
    np.testing.assert_allclose(out["inv_rms"], 1.0 / np.sqrt(c * c + 1e-6), rtol=1e-14)


def test_pre_mixes_brute_force(rng):
    T, N, D = 2, 4, 3
    x, phi, alpha, base = _pre_inputs(rng, T, N, D)
    out = orc.pre_fwd(x, phi, alpha, base)
    M = phi.shape[0]
    for t in range(T):
        ss = sum(x[t, n, d] ** 2 for n in range(N) for d in range(D))
        inv = 1.0 / np.sqrt(ss / (N * D) + 1e-6)
        for m in range(M):
            want = sum(x[t, n, d] * inv * phi[m, n * D + d] for n in range(N) for d in range(D))
            assert abs(out["mixes"][t, m] - want) < 1e-12


@pytest.mark.parametrize("N", [4, 8])
def test_pre_sigmoid_identity_and_y(rng, N):
    T, D = 3, 6
    M = 2 * N + N * N
    x = rng.standard_normal((T, N, D))
    eps = 1e-3
    out = orc.pre_fwd(x, np.zeros((M, N * D)), np.ones(3), np.zeros(M), hc_eps=eps, iter_times=5)
    np.testing.assert_allclose(out["pre"], 0.5 + eps, rtol=1e-15)
    np.testing.assert_allclose(out["post_out"], 1.0, rtol=1e-15)
    assert not out["h_res_logits"].any()
    # y = sum_n pre_n x_n with pre = 0.5 + eps
    for t, d in itertools.product(range(T), range(D)):
        assert abs(out["y"][t, d] - sum((0.5 + eps) * x[t, n, d] for n in range(N))) < 1e-12
    # base alone sets the heads
    base = rng.standard_normal(M)
    out = orc.pre_fwd(x, np.zeros((M, N * D)), np.ones(3), base, hc_eps=eps)
    np.testing.assert_allclose(out["pre"], np.tile(_sig(base[:N]) + eps, (T, 1)), rtol=1e-14)
    np.testing.assert_allclose(out["post_out"], np.tile(2 * _sig(base[N:2 * N]), (T, 1)), rtol=1e-14)


def test_pre_clamp_saturation(rng):
    T, N, D = 2, 4, 4
    M = 2 * N + N * N
    x = rng.standard_normal((T, N, D))
    base = np.zeros(M)
    base[2 * N:] = np.linspace(-40, 40, N * N)
    out = orc.pre_fwd(x, np.zeros((M, N * D)), np.ones(3), base, clamp_min=-3.0, clamp_max=3.0)
    base_c = base.copy()
    base_c[2 * N:] = np.clip(base_c[2 * N:], -3, 3)
    out_c = orc.pre_fwd(x, np.zeros((M, N * D)), np.ones(3), base_c)
    np.testing.assert_allclose(out["comb_frag"], out_c["comb_frag"], rtol=1e-14)
    np.testing.assert_array_equal(out["h_res_logits"].reshape(T, -1), np.broadcast_to(base[2 * N:], (T, N * N)))
    # (0, 0) disables the clamp: logits of +-40 then dominate the softmax
    out_off = orc.pre_fwd(x, np.zeros((M, N * D)), np.ones(3), base)
    assert np.abs(out_off["comb_frag"] - out["comb_frag"]).max() > 1e-2


# ---------------------------------------------------------------------------
# pre backward: finite differences of the scalar loss
# ---------------------------------------------------------------------------
def _pre_loss(x, phi, alpha, base, gy, gpost, gcomb, **kw):
    out = orc.pre_fwd(x, phi, alpha, base, **kw)
    return float((out["y"] * gy).sum() + (out["post_out"] * gpost).sum()
                 + (out["comb_frag"] * gcomb).sum())


CASES = [
    dict(N=4, clamp=(0.0, 0.0), iters=20, eps=1e-6),
    dict(N=4, clamp=(-0.4, 0.4), iters=20, eps=1e-6),
    dict(N=4, clamp=(0.0, 0.0), iters=1, eps=1e-2),
    dict(N=8, clamp=(-0.5, 0.5), iters=7, eps=1e-3),
    dict(N=2, clamp=(0.0, 0.0), iters=4, eps=1e-6),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"N{c['N']}-it{c['iters']}-clamp{c['clamp'][1]}")
def test_pre_bwd_finite_differences(rng, case):
    N, (cmin, cmax), iters, heps = case["N"], case["clamp"], case["iters"], case["eps"]
    T, D = 3, 5
    x, phi, alpha, base = _pre_inputs(rng, T, N, D, phi_scale=0.8)
    gy = rng.standard_normal((T, D))
    gpost = rng.standard_normal((T, N))
    gcomb = rng.standard_normal((T, N, N))
    kw = dict(norm_eps=1e-6, hc_eps=heps, clamp_min=cmin, clamp_max=cmax, iter_times=iters)
    if cmax:
        logits = orc.pre_fwd(x, phi, alpha, base, **kw)["h_res_logits"]
        inside = (logits > cmin) & (logits < cmax)
        assert inside.any() and (~inside).any()           # both gradient paths exercised
        assert np.min(np.abs(np.abs(logits) - cmax)) > 1e-3  # FD does not straddle a bound
    grads = orc.pre_bwd(x, phi, alpha, base, gy, gpost, gcomb, **kw)
    args = (x, phi, alpha, base)
    f = lambda *a: _pre_loss(*a, gy, gpost, gcomb, **kw)
    for idx in range(4):
        for _ in range(2):
            v = rng.standard_normal(args[idx].shape)
            want = _fd(f, args, idx, v, eps=1e-6)
            got = float((grads[idx] * v).sum())
            assert abs(got - want) <= 2e-6 * (1 + abs(want)), (idx, got, want)
    # every coordinate of alpha and base
    for idx in (2, 3):
        for c in range(args[idx].size):
            v = np.zeros(args[idx].shape)
            v.flat[c] = 1.0
            want = _fd(f, args, idx, v, eps=1e-6)
            assert abs(grads[idx].flat[c] - want) <= 2e-6 * (1 + abs(want)), (idx, c)
