"""The single-pass pre forward (one HBM read of x; N = 4, bf16 x and phi,
D = 4096 or 7168 .. 8192, T >= 8192) that mhc_pre_fwd takes when the
caller's workspace holds its exchange ring, called through the C ABI.

Checked against
  * the two-pass forms, run by mhc_pre_fwd with a 4 MiB workspace (enough
    for them, too small for the single-pass exchange ring), over every
    token: the sums are added in other orders, so the fp32 outputs agree to
    accumulation rounding and y to bf16 rounding;
  * the float64 oracle on a token subset (first, last, random, ragged tail);
  * itself: a second call is bit-identical (fixed reduction order), and so
    is mhc_pre_fwd_noalloc, whose 64 MiB scratch has room for the ring.
The control words at the start of the workspace's single-pass region show
that the path ran (every block registered), and the status word of
mhc_pre_fwd_ex (pinned host memory the kernels write) that no bounded wait
timed out (status 0).  A forced timeout (the waits' limit set to zero through
the mhc_debug_set_wait_limit test hook) must surface as a nonzero status and
as a RuntimeError from the package's operators."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from FlagOS_mhc import _lib
from oracle import mhc_oracle as orc

pytestmark = pytest.mark.gpu
DEV = "cuda"
CTL = 256          # byte offset of the single-pass control words in the workspace
ARRIVED, STATUS = 16, 17
STATUS_OUT = 63    # (test only) where _run puts mhc_pre_fwd_ex's status word


def _inputs(T, N, D, seed):
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    M = 2 * N + N * N
    x = torch.randn(T, N, D, device=DEV, generator=g).to(torch.bfloat16)
    phi = (torch.randn(M, N * D, device=DEV, generator=g) / (N * D) ** 0.5).to(torch.bfloat16)
    alpha = torch.tensor([0.5, 0.5, 1.0], device=DEV)
    base = torch.randn(M, device=DEV, generator=g) * 0.1
    return x, phi, alpha, base


TWO_PASS_WS = 4 << 20


def _run(mode, x, phi, alpha, base, xs, clamp=10.0, iters=20):
    """mode: "full" (mhc_pre_fwd, its workspace size), "two-pass" (mhc_pre_fwd,
    TWO_PASS_WS bytes) or "noalloc"."""
    T, N, D = x.shape
    M = 2 * N + N * N
    f32 = dict(device=DEV, dtype=torch.float32)
    o = {"y": torch.empty(T, D, device=DEV, dtype=x.dtype), "post_out": torch.empty(T, N, **f32),
         "comb_frag": torch.empty(T, N, N, **f32), "inv_rms": torch.empty(T, **f32),
         "mixes": torch.empty(T, M, **f32), "h_res_logits": torch.empty(T, N, N, **f32),
         "pre": torch.empty(T, N, **f32), "x_scaled": torch.empty(T, N * D, **f32) if xs else None}
    lib = _lib.load()
    head = (x.data_ptr(), 1, phi.data_ptr(), 1, alpha.data_ptr(), base.data_ptr(), 1e-6, 1e-6,
            -clamp, clamp, iters) + tuple(_lib.ptr(o[k]) for k in o)
    stream = torch.cuda.current_stream().cuda_stream
    ws = None
    status = torch.full((1,), -7, dtype=torch.int32, pin_memory=True)  # the kernels overwrite it
    if mode == "noalloc":
        rc = lib.mhc_pre_fwd_noalloc(*head, T, N, D, stream)
    else:
        full = lib.mhc_pre_fwd_workspace_size(T, N, D, 1)
        if mode == "two-pass":
            assert TWO_PASS_WS < full  # the single-pass form would need more
        ws = torch.zeros(full if mode == "full" else TWO_PASS_WS, dtype=torch.uint8, device=DEV)
        rc = lib.mhc_pre_fwd_ex(*head, ws.data_ptr(), ws.numel(), status.data_ptr(), T, N, D, stream)
    _lib.check(rc, mode)
    torch.cuda.synchronize()
    ctl = ws[CTL:CTL + 256].view(torch.int32).cpu().numpy() if ws is not None else None
    if ctl is not None:
        ctl = ctl.copy()
        ctl[STATUS_OUT] = int(status[0])  # the caller's copy of the status word
    return o, ctl


CASES = [
    # (T, D, x_scaled)
    (8192, 7168, False),     # 28 members a group
    (8200, 7168, False),     # ragged last tile, groups with unequal tile counts
    (8200, 7168, True),      # with fp32 x_scaled (loads two tiles ahead)
    (16384, 4096, False),    # two groups per XCC
    (16390, 4096, True),     # ragged, with fp32 x_scaled
    (8192, 7680, False),     # 256-column slices, 30 members a group
    (8192, 8192, True),      # 256-column slices, 32 members a group, x_scaled
    (65536, 7168, False),    # BASELINE config 5 width and length
]


@pytest.mark.parametrize("T,D,xs", CASES, ids=[f"T{t}-D{d}{'-xs' if s else ''}" for t, d, s in CASES])
def test_single_pass_matches_two_pass_and_oracle(T, D, xs):
    N = 4
    x, phi, alpha, base = _inputs(T, N, D, seed=T + D)
    sp, ctl = _run("full", x, phi, alpha, base, xs)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    assert ctl[ARRIVED] == cus, f"single-pass path did not run: {ctl[ARRIVED]} of {cus} blocks registered"
    assert ctl[STATUS] == 0, f"a bounded wait timed out (status {ctl[STATUS]})"
    assert ctl[STATUS_OUT] == 0, "the caller's status word was not written"
    tp, ctl_tp = _run("two-pass", x, phi, alpha, base, xs)
    assert ctl_tp[STATUS_OUT] == -7, "the two-pass forms leave the status word alone"
    # two-pass vs single-pass: fp32 sums in other orders
    for k, atol, rtol in (("mixes", 2e-4, 1e-4), ("inv_rms", 0.0, 2e-5), ("pre", 1e-5, 1e-5),
                          ("post_out", 1e-5, 1e-5), ("comb_frag", 1e-5, 1e-5), ("h_res_logits", 2e-4, 1e-4)):
        err = (sp[k] - tp[k]).abs()
        bound = atol + rtol * tp[k].abs()
        assert bool((err <= bound).all()), f"{k}: max err {float(err.max()):.3e}"
    # y: bf16 outputs of pre values that differ by accumulation rounding
    assert torch.allclose(sp["y"].float(), tp["y"].float(), rtol=1e-2, atol=1e-2)
    if xs:
        assert torch.allclose(sp["x_scaled"], tp["x_scaled"], rtol=2e-5, atol=1e-6)
    # the oracle on a token subset
    rng = np.random.default_rng(T)
    idx = np.unique(np.r_[0, T - 1, T - 2, rng.integers(0, T, 32)])
    it = torch.from_numpy(idx).to(DEV)
    f = lambda t: t.detach().double().cpu().numpy()
    want = orc.pre_fwd(f(x[it]), f(phi), f(alpha), f(base), norm_eps=1e-6, hc_eps=1e-6,
                       clamp_min=-10.0, clamp_max=10.0, iter_times=20)
    for k, tol in (("mixes", 1e-4), ("inv_rms", 1e-5), ("pre", 1e-5), ("post_out", 1e-5),
                   ("comb_frag", 1e-5), ("h_res_logits", 1e-4)):
        np.testing.assert_allclose(f(sp[k][it]), want[k], rtol=tol, atol=tol, err_msg=k)
    np.testing.assert_allclose(f(sp["y"][it]), want["y"], rtol=2e-2, atol=2e-2, err_msg="y")
    if xs:
        np.testing.assert_allclose(f(sp["x_scaled"][it]), want["x_scaled"], rtol=1e-5, atol=1e-5)
    # fixed reduction order: a second call is bit-identical
    sp2, ctl2 = _run("full", x, phi, alpha, base, xs)
    assert ctl2[STATUS] == 0
    na, _ = _run("noalloc", x, phi, alpha, base, xs)
    for k in sp:
        if sp[k] is not None:
            assert torch.equal(sp[k], sp2[k]), k
            assert torch.equal(sp[k], na[k]), "noalloc " + k


def test_two_pass_workspace_is_not_the_single_pass():
    """The 4 MiB workspace really selects the two-pass forms: their sums run
    in another order, so some mixes differ from the single-pass ones in
    rounding (and only in rounding)."""
    T, N, D = 8192, 4, 7168
    x, phi, alpha, base = _inputs(T, N, D, seed=5)
    sp, _ = _run("full", x, phi, alpha, base, False)
    tp, _ = _run("two-pass", x, phi, alpha, base, False)
    assert not torch.equal(sp["mixes"], tp["mixes"])
    assert torch.allclose(sp["mixes"], tp["mixes"], rtol=1e-4, atol=2e-4)


def test_single_pass_failure_is_loud():
    """With the waits' limit forced to zero ticks from the host (the
    mhc_debug_set_wait_limit test hook), the single-pass kernel gives up at
    its first unsatisfied wait and every kernel still exits: the status word
    is set, every output of the call is NaN, never silently wrong, and the
    package's operators raise RuntimeError (check_errors, the next forward,
    and the backward of an autograd forward that failed).  With the normal
    limit restored the next call is correct again."""
    import FlagOS_mhc as m

    T, N, D = 8192, 4, 7168
    x, phi, alpha, base = _inputs(T, N, D, seed=9)
    lib = _lib.load()
    good, ctl = _run("full", x, phi, alpha, base, True)
    assert ctl[STATUS] == 0 and ctl[STATUS_OUT] == 0
    m.check_errors()  # nothing pending that failed
    try:
        lib.mhc_debug_set_wait_limit(0)
        bad, ctl_bad = _run("full", x, phi, alpha, base, True)
        assert ctl_bad[STATUS] != 0
        assert ctl_bad[STATUS_OUT] == ctl_bad[STATUS], "the caller's status word carries the failure"
        for k, v in bad.items():
            assert bool(torch.isnan(v.float()).all()), k
        # the package: the call itself returns (its kernels have not run yet) ...
        out = m.mhc_pre_clamp_sinkhorn(x, phi, alpha, base, clamp_min=-10.0, clamp_max=10.0)
        torch.cuda.synchronize()
        assert bool(torch.isnan(out["y"].float()).all())
        # ... and the failure is raised at the next check
        with pytest.raises(RuntimeError, match="bounded wait"):
            m.check_errors()
        m.check_errors()  # reported once
        # the next forward raises for an earlier failed call whose work has finished
        m.mhc_pre_clamp_sinkhorn(x, phi, alpha, base, clamp_min=-10.0, clamp_max=10.0)
        torch.cuda.synchronize()
        with pytest.raises(RuntimeError, match="bounded wait"):
            m.mhc_pre_clamp_sinkhorn(x[:64], phi, alpha, base)
        # the backward of a failed autograd forward raises instead of propagating NaN
        xg = x.clone().requires_grad_(True)
        y, po, cf = m.mhc_pre_clamp_sinkhorn_fn(xg, phi, alpha, base, clamp_min=-10.0, clamp_max=10.0)
        with pytest.raises(RuntimeError, match="bounded wait"):
            (y.float().sum() + po.sum() + cf.sum()).backward()
    finally:
        lib.mhc_debug_set_wait_limit(-1)
        torch.cuda.synchronize()
    m.check_errors()
    again, ctl2 = _run("full", x, phi, alpha, base, True)
    assert ctl2[STATUS] == 0 and ctl2[STATUS_OUT] == 0
    for k in good:
        assert torch.equal(good[k], again[k]), k
