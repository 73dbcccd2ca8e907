"""Golden fixtures (tests/golden/mhc_golden.npz, written by make_golden.py from
the oracle).  CPU: the oracle still reproduces them.  GPU: the HIP operators
match them (fixtures as the parity reference, same tolerances as the other
GPU parity tests)."""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from oracle import mhc_oracle as orc

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "mhc_golden.npz")


def _cases(prefix):
    z = np.load(GOLDEN)
    names = sorted({k.split("/")[0] for k in z.files if k.startswith(prefix)})
    return [(n, {k.split("/", 1)[1]: z[k] for k in z.files if k.startswith(n + "/")}) for n in names]


POST = _cases("post_")
PRE = _cases("pre_")


def _kw(c):
    ne, he, cmin, cmax, it = c["hyper"].tolist()
    return dict(norm_eps=ne, hc_eps=he, clamp_min=cmin, clamp_max=cmax, iter_times=int(it))


@pytest.mark.parametrize("name,c", POST, ids=[n for n, _ in POST])
def test_oracle_reproduces_post_golden(name, c):
    np.testing.assert_allclose(orc.post_fwd(c["x"], c["h_res"], c["h_out"], c["h_post"]), c["y"],
                               rtol=1e-12, atol=1e-12)
    got = orc.post_bwd(c["grad_y"], c["x"], c["h_res"], c["h_out"], c["h_post"])
    for g, k in zip(got, ("grad_x", "grad_h_res", "grad_h_out", "grad_h_post")):
        np.testing.assert_allclose(g, c[k], rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("name,c", PRE, ids=[n for n, _ in PRE])
def test_oracle_reproduces_pre_golden(name, c):
    kw = _kw(c)
    fwd = orc.pre_fwd(c["x"], c["phi"], c["alpha"], c["base"], **kw)
    for k, v in fwd.items():
        np.testing.assert_allclose(v, c["fwd_" + k], rtol=1e-12, atol=1e-12)
    got = orc.pre_bwd(c["x"], c["phi"], c["alpha"], c["base"], c["grad_y"], c["grad_post_out"],
                      c["grad_comb_frag"], **kw)
    for g, k in zip(got, ("grad_x", "grad_phi", "grad_alpha", "grad_base")):
        np.testing.assert_allclose(g, c[k], rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------------------------
# GPU: HIP operators against the fixtures
# ---------------------------------------------------------------------------
def _t(a, dtype):
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda").to(dtype)


def _close(got, want, rtol, atol, what):
    got = got.detach().double().cpu().numpy()
    err = np.abs(got - want)
    bad = err > atol + rtol * np.abs(want)
    assert not bad.any(), f"{what}: {bad.sum()}/{bad.size} outside tol, max err {err.max():.3e}"


@pytest.mark.gpu
@pytest.mark.parametrize("name,c", POST, ids=[n for n, _ in POST])
def test_gpu_post_golden(name, c):
    import FlagOS_mhc as m
    bf = torch.bfloat16
    x, hr, ho, hp, gy = (_t(c["x"], bf), _t(c["h_res"], torch.float32), _t(c["h_out"], bf),
                         _t(c["h_post"], torch.float32), _t(c["grad_y"], bf))
    _close(m.mhc_post(x, hr, ho, hp), c["y"], 2e-2, 2e-2, "y")
    gx, ghr, gho, ghp = m.mhc_post_backward(gy, x, hr, ho, hp)
    _close(gx, c["grad_x"], 2e-2, 2e-2, "grad_x")
    _close(gho, c["grad_h_out"], 2e-2, 2e-2, "grad_h_out")
    _close(ghr, c["grad_h_res"], 1e-4, 1e-4 * np.abs(c["grad_h_res"]).max(), "grad_h_res")
    _close(ghp, c["grad_h_post"], 1e-4, 1e-4 * np.abs(c["grad_h_post"]).max(), "grad_h_post")


@pytest.mark.gpu
@pytest.mark.parametrize("name,c", PRE, ids=[n for n, _ in PRE])
def test_gpu_pre_golden(name, c):
    import FlagOS_mhc as m
    bf = torch.bfloat16
    kw = _kw(c)
    x = _t(c["x"], bf)
    phi = _t(c["phi"], bf if name != "pre_ref_test" and name != "pre_iter1_n4" else torch.float32)
    alpha, base = _t(c["alpha"], torch.float32), _t(c["base"], torch.float32)
    out = m.mhc_pre_clamp_sinkhorn(x, phi, alpha, base, need_backward=True, **kw)
    _close(out["y"], c["fwd_y"], 2e-2, 2e-2, "y")
    for k in ("post_out", "comb_frag", "inv_rms", "mixes", "h_res_logits", "pre"):
        _close(out[k], c["fwd_" + k], 1e-4, 1e-5, k)
    gx, gphi, ga, gb = m.mhc_pre_clamp_sinkhorn_backward(
        x, phi, alpha, base, out["inv_rms"], out["x_scaled"], out["mixes"], out["h_res_logits"],
        out["pre"], _t(c["grad_y"], bf), _t(c["grad_post_out"], torch.float32),
        _t(c["grad_comb_frag"], torch.float32), **kw)
    _close(gx, c["grad_x"], 2e-2, 2e-2, "grad_x")
    for got, k in ((gphi, "grad_phi"), (ga, "grad_alpha"), (gb, "grad_base")):
        _close(got, c[k], 1e-4, 1e-5 * np.abs(c[k]).max(), k)
