"""The single-pass pre backward (x and grad_y read from HBM once; N = 4, bf16
x, grad_y and phi, D = 4096 or 7168 .. 8192, T >= 8192), which
mhc_pre_bwd_ex runs unless MHC_PRE_BWD_TWO_PASS is set (also with
MHC_PRE_BWD_SINGLE_PASS), called through the C ABI and through the package.

Checked against
  * the two-pass forms (MHC_PRE_BWD_TWO_PASS) over every token: grad_pre is
    summed in another order, so grad_x agrees to bf16 rounding and the fp32
    T-reductions to accumulation rounding;
  * a float64 reference over all tokens (gpu_ref.pre_bwd_fp64: grad_x at the
    bf16 tolerance, grad_phi / grad_alpha / grad_base at rtol 1e-4 with atol
    1e-5 * max|ref|) and the float64 oracle on a token subset;
  * itself: a second call is bit-identical (fixed reduction orders).
The status word of mhc_pre_bwd_ex (pinned host memory, written by the
kernels) shows that the single pass ran (0; the two-pass forms leave it
untouched) and that no bounded wait timed out.  A forced timeout (waits'
limit zero through mhc_debug_set_wait_limit) must give a nonzero status,
NaN outputs and a RuntimeError from the package."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import FlagOS_mhc as m
from FlagOS_mhc import _lib
from FlagOS_mhc.mhc_pre_clamp_sinkhorn_backward import _pre_backward
from gpu_ref import check_reductions, close_gpu, pre_bwd_fp64
from oracle import mhc_oracle as orc
from test_gpu_post import DEV, _np, _subset, assert_close
from test_gpu_pre import pre_inputs

pytestmark = pytest.mark.gpu

KW = dict(norm_eps=1e-6, hc_eps=1e-6, clamp_min=-10.0, clamp_max=10.0, iter_times=20)
UNTOUCHED = -7


def _bwd_abi(x, phi, alpha, base, fwd, gy, gpost, gcomb, two_pass, flags=None):
    """mhc_pre_bwd_ex through ctypes (MHC_PRE_BWD_TWO_PASS or
    MHC_PRE_BWD_SINGLE_PASS unless `flags` is given); returns the outputs and
    the status word."""
    T, N, D = x.shape
    M = 2 * N + N * N
    lib = _lib.load()
    gx = torch.empty_like(x)
    gphi = torch.empty(M, N * D, device=DEV)
    ga = torch.empty(3, device=DEV)
    gb = torch.empty(M, device=DEV)
    ws_bytes = lib.mhc_pre_bwd_workspace_size(T, N, D, 1, KW["iter_times"])
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=DEV)
    status = torch.full((1,), UNTOUCHED, dtype=torch.int32, pin_memory=True)
    rc = lib.mhc_pre_bwd_ex(
        x.data_ptr(), 1, phi.data_ptr(), 1, alpha.data_ptr(), base.data_ptr(), fwd["inv_rms"].data_ptr(),
        fwd["mixes"].data_ptr(), fwd["pre"].data_ptr(), gy.data_ptr(), gpost.data_ptr(), gcomb.data_ptr(),
        KW["hc_eps"], KW["clamp_min"], KW["clamp_max"], KW["iter_times"], None, gx.data_ptr(), gphi.data_ptr(),
        ga.data_ptr(), gb.data_ptr(),
        flags if flags is not None else (_lib.PRE_BWD_TWO_PASS if two_pass else _lib.PRE_BWD_SINGLE_PASS),
        status.data_ptr(),
        ws.data_ptr(), ws_bytes, T, N, D, torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "mhc_pre_bwd_ex")
    torch.cuda.synchronize()
    return (gx, gphi, ga, gb), int(status[0])


CASES = [
    # (T, D)
    (8192, 7168),     # fewest tokens the single pass takes
    (8200, 7168),     # ragged last tile, groups with unequal tile counts
    (16384, 4096),    # BASELINE config 3 shape: two groups per XCC
    (16390, 8192),    # 32 members a group, ragged
    (65536, 7168),
]


@pytest.mark.parametrize("T,D", CASES, ids=[f"T{t}-D{d}" for t, d in CASES])
def test_single_pass_bwd_parity(T, D):
    print(f"[pre_bwd single pass] T={T} N=4 D={D}", flush=True)
    N = 4
    x, phi, alpha, base, gy, gpost, gcomb = pre_inputs(T, N, D, seed=T + D)
    fwd = m.mhc_pre_clamp_sinkhorn(x, phi, alpha, base, need_backward=True, **KW)
    sp, st = _bwd_abi(x, phi, alpha, base, fwd, gy, gpost, gcomb, two_pass=False)
    assert st == 0, f"single pass did not run or a bounded wait timed out (status {st})"
    tp, st2 = _bwd_abi(x, phi, alpha, base, fwd, gy, gpost, gcomb, two_pass=True)
    assert st2 == UNTOUCHED, "the two-pass forms leave the status word alone"
    # single vs two-pass: grad_pre summed in other orders
    close_gpu(sp[0].float(), tp[0].float(), 2e-2, 2e-2, "grad_x single vs two-pass")
    for got, want, name in zip(sp[1:], tp[1:], ("grad_phi", "grad_alpha", "grad_base")):
        close_gpu(got, want, 1e-4, 1e-5 * float(want.abs().max()), name + " single vs two-pass")
    # float64 reference over every token, the oracle on a subset
    ref = pre_bwd_fp64(x, phi, alpha, base, gy, gpost, gcomb, KW, grad_x=sp[0])
    check_reductions(sp[1], sp[2], sp[3], ref, "single pass")
    idx = _subset(T)
    sub = orc.pre_bwd(_np(x[idx]), _np(phi), _np(alpha), _np(base), _np(gy[idx]), _np(gpost[idx]),
                      _np(gcomb[idx]), **KW)
    assert_close(sp[0][idx], sub[0], 2e-2, 2e-2, "grad_x subset vs oracle")
    # fixed reduction orders: a second call gives the same bits
    sp2, st3 = _bwd_abi(x, phi, alpha, base, fwd, gy, gpost, gcomb, two_pass=False)
    assert st3 == 0
    for a, b in zip(sp, sp2):
        assert torch.equal(a, b)


def test_single_pass_bwd_through_package():
    """Without a pass flag the library takes the single pass from T = 8192
    (status 0) and the two-pass forms below (status untouched); the
    package's backward (single_pass=None) equals the ABI call bit for bit,
    single_pass=False the two-pass forms and single_pass=True the single
    pass where it applies."""
    N, D = 4, 7168
    for T, auto_single in ((8192, True), (4096, False)):
        x, phi, alpha, base, gy, gpost, gcomb = pre_inputs(T, N, D, seed=3)
        fwd = m.mhc_pre_clamp_sinkhorn(x, phi, alpha, base, need_backward=True, **KW)
        got = m.mhc_pre_clamp_sinkhorn_backward(x, phi, alpha, base, fwd["inv_rms"], None, fwd["mixes"], None,
                                                fwd["pre"], gy, gpost, gcomb, **KW)
        auto, st = _bwd_abi(x, phi, alpha, base, fwd, gy, gpost, gcomb, two_pass=False, flags=0)
        assert st == (0 if auto_single else UNTOUCHED)
        for a, b in zip(got, auto):
            assert torch.equal(a.reshape(b.shape), b)
        kw = (KW["norm_eps"], KW["hc_eps"], KW["clamp_min"], KW["clamp_max"], KW["iter_times"])
        for sp in (False, True):
            pkg = _pre_backward(x, phi, alpha, base, fwd["inv_rms"], fwd["mixes"], fwd["pre"], gy, gpost, gcomb,
                                *kw, single_pass=sp)
            abi, st = _bwd_abi(x, phi, alpha, base, fwd, gy, gpost, gcomb, two_pass=not sp)
            assert st == (0 if sp and auto_single else UNTOUCHED)
            for a, b in zip(pkg, abi):
                assert torch.equal(a.reshape(b.shape), b)
        del x, gy, fwd, got, auto, pkg, abi
    m.check_errors()


def test_single_pass_bwd_failure_is_loud():
    """With the waits' limit forced to zero ticks from the host, the single
    pass gives up at its first unsatisfied wait and every kernel still exits:
    the status word is set, grad_x / grad_phi / grad_alpha / grad_base are
    NaN, and the package raises RuntimeError.  With the normal limit restored
    the next call is correct again."""
    T, N, D = 8192, 4, 7168
    x, phi, alpha, base, gy, gpost, gcomb = pre_inputs(T, N, D, seed=11)
    fwd = m.mhc_pre_clamp_sinkhorn(x, phi, alpha, base, need_backward=True, **KW)
    good, st = _bwd_abi(x, phi, alpha, base, fwd, gy, gpost, gcomb, two_pass=False)
    assert st == 0
    lib = _lib.load()
    try:
        lib.mhc_debug_set_wait_limit(0)
        bad, st_bad = _bwd_abi(x, phi, alpha, base, fwd, gy, gpost, gcomb, two_pass=False)
        assert st_bad > 0
        for v in bad:
            assert bool(torch.isnan(v.float()).all())
        _pre_backward(x, phi, alpha, base, fwd["inv_rms"], fwd["mixes"], fwd["pre"], gy, gpost, gcomb,
                      KW["norm_eps"], KW["hc_eps"], KW["clamp_min"], KW["clamp_max"], KW["iter_times"],
                      single_pass=True)
        with pytest.raises(RuntimeError, match="bounded wait"):
            m.check_errors()
    finally:
        lib.mhc_debug_set_wait_limit(-1)
        torch.cuda.synchronize()
    m.check_errors()
    again, st2 = _bwd_abi(x, phi, alpha, base, fwd, gy, gpost, gcomb, two_pass=False)
    assert st2 == 0
    for a, b in zip(good, again):
        assert torch.equal(a, b)
