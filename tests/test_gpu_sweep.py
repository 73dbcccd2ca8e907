"""Seeded sweep over random shapes: every operator (mhc_post, its backward,
mhc_pre_clamp_sinkhorn, its backward, and the fused post + pre forward) on
shapes drawn around the kernel-selection thresholds (T = 1024 for the
streaming post kernels, T = 16384 for the split grad_pre, D = 256 / 5120 for
the fused and block-per-token kernels, D % 8 and D % 64 for the vector and
LDS-pipelined forms), so that shapes no hand-written case names still meet
the float64 oracle.

Tolerances are the north-star ones used by the per-operator tests: bf16 /
fp16 outputs rtol 2e-2 / atol 2e-2, fp32 per-token outputs rtol 1e-4 (atol
1e-5), fp32 token reductions rtol 1e-4 with atol 1e-5 * max|ref|.  Per-token
outputs are checked against the oracle on a token subset; grad_phi,
grad_alpha and grad_base over all tokens against the float64 reference of
gpu_ref.pre_bwd_fp64 (device contractions, oracle small stage) at rtol 1e-4
with atol 1e-5 * max|ref|."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import FlagOS_mhc as m
from gpu_ref import check_reductions, pre_bwd_fp64
from oracle import mhc_oracle as orc
from test_gpu_post import DEV, _np, _subset, assert_close, post_inputs, tol_for
from test_gpu_pre import FWD_KEYS, _oracle_fwd, check_fwd, pre_inputs

pytestmark = pytest.mark.gpu

_DT = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}


def _cases(n=40, seed=2026):
    r = np.random.default_rng(seed)
    out = []
    for i in range(n):
        N = int(r.choice([4, 4, 4, 8]))
        dt = str(r.choice(["bf16", "bf16", "bf16", "f16", "f32"]))
        phi_dt = dt if dt != "f16" or r.random() < 0.5 else "f32"
        if dt == "bf16" and r.random() < 0.3:
            phi_dt = "f32"
        # D: multiples of 64 (fused / LDS-pipelined), of 8 (vector), or ragged
        kind = r.random()
        if kind < 0.5:
            D = 64 * int(r.integers(2, 130))
        elif kind < 0.8:
            D = 8 * int(r.integers(1, 700))
        else:
            D = int(r.integers(1, 3000))
        # T: around the thresholds or small
        tk = r.random()
        if tk < 0.35:
            T = int(r.integers(1, 130))
        elif tk < 0.7:
            T = int(r.choice([1023, 1024, 1025])) + int(r.integers(-3, 4))
        else:
            T = int(r.integers(130, 2600))
        T = max(1, min(T, (48 << 20) // (N * D)))   # keep x under ~96 MB (bf16)
        clamp = float(r.choice([0.0, 0.5, 3.0, 10.0]))
        iters = int(r.choice([1, 7, 20, 33]))
        out.append((i, T, N, D, dt, phi_dt, clamp, iters))
    return out


CASES = _cases() + [
    (40, 1024, 4, 5120, "bf16", "bf16", 10.0, 20),    # block-per-token post kernels, fused forward
    (41, 1100, 4, 9216, "bf16", "bf16", 3.0, 20),
    (42, 16384, 4, 704, "bf16", "bf16", 10.0, 20),    # grad_pre in kernel A (T >= 16384)
    (43, 16383, 4, 768, "bf16", "f32", 10.0, 20),     # split grad_pre, two phi planes
]


@pytest.mark.parametrize("i,T,N,D,dt,phi_dt,clamp,iters", CASES)
def test_sweep(i, T, N, D, dt, phi_dt, clamp, iters):
    dtype, phi_dtype = _DT[dt], _DT[phi_dt]
    tag = f"[sweep {i}] T={T} N={N} D={D} {dt} phi={phi_dt} clamp={clamp} it={iters}"
    idx = _subset(T, k=24, seed=i)
    rtol, atol = tol_for(dtype)

    print(tag, "post", flush=True)
    x, h_res, h_out, h_post, gyp = post_inputs(T, N, D, dtype, seed=100 + i)
    y = m.mhc_post(x, h_res, h_out, h_post)
    gx, ghr, gho, ghp = m.mhc_post_backward(gyp, x, h_res, h_out, h_post)
    torch.cuda.synchronize()
    assert_close(y[idx], orc.post_fwd(_np(x[idx]), _np(h_res[idx]), _np(h_out[idx]), _np(h_post[idx])),
                 rtol, atol, tag + " post y")
    w = orc.post_bwd(_np(gyp[idx]), _np(x[idx]), _np(h_res[idx]), _np(h_out[idx]), _np(h_post[idx]))
    assert_close(gx[idx], w[0], rtol, atol, tag + " post grad_x")
    assert_close(gho[idx], w[2], rtol, atol, tag + " post grad_h_out")
    assert_close(ghr[idx], w[1], 1e-4, 1e-4 * np.abs(w[1]).max(), tag + " post grad_h_res")
    assert_close(ghp[idx], w[3], 1e-4, 1e-4 * np.abs(w[3]).max(), tag + " post grad_h_post")

    print(tag, "pre", flush=True)
    xp, phi, alpha, base, gy, gpost, gcomb = pre_inputs(T, N, D, dtype, phi_dtype, seed=200 + i)
    kw = dict(norm_eps=1e-6, hc_eps=1e-6, clamp_min=-clamp, clamp_max=clamp, iter_times=iters)
    out = m.mhc_pre_clamp_sinkhorn(xp, phi, alpha, base, need_backward=True, **kw)
    torch.cuda.synchronize()
    check_fwd(out, _oracle_fwd(idx, xp, phi, alpha, base, kw), dtype, idx, tag + " pre:")
    g = m.mhc_pre_clamp_sinkhorn_backward(xp, phi, alpha, base, out["inv_rms"], out["x_scaled"], out["mixes"],
                                          out["h_res_logits"], out["pre"], gy, gpost, gcomb, **kw)
    torch.cuda.synchronize()
    sub = orc.pre_bwd(_np(xp[idx]), _np(phi), _np(alpha), _np(base), _np(gy[idx]), _np(gpost[idx]),
                      _np(gcomb[idx]), **kw)
    assert_close(g[0][idx], sub[0], 2e-2, 2e-2, tag + " pre grad_x")
    ref = pre_bwd_fp64(xp, phi, alpha, base, gy, gpost, gcomb, kw)
    check_reductions(g[1], g[2], g[3], ref, tag + " pre")

    print(tag, "post_pre", flush=True)
    pkw = dict(kw)
    x_next, fo = m.mhc_post_pre_clamp_sinkhorn(x, h_res, h_out, h_post, phi, alpha, base,
                                               need_backward=True, **pkw)
    unf = m.mhc_pre_clamp_sinkhorn(y, phi, alpha, base, need_backward=True, **pkw)
    torch.cuda.synchronize()
    assert torch.equal(x_next, y), tag + " x_next differs from mhc_post"
    check_fwd(fo, _oracle_fwd(idx, y, phi, alpha, base, kw), dtype, idx, tag + " post_pre:")
    for k in FWD_KEYS:
        a, b = fo[k].float(), unf[k].float()
        tol = 1e-5 + 1e-4 * float(b.abs().max()) + 1e-4 * b.abs()
        assert bool(((a - b).abs() <= tol).all()), tag + " post_pre " + k + " vs unfused"
