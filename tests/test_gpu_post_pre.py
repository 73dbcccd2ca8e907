"""GPU parity of the fused forward mhc_post_pre_clamp_sinkhorn (mhc_post of
layer l, then mhc_pre_clamp_sinkhorn of layer l+1 on its output).

x_next must be bit-identical to mhc_post (same fp32 FMA order and rounding).
The pre outputs are checked against the float64 oracle applied to that
x_next on a token subset (bf16 y rtol/atol 2e-2, fp32 outputs rtol 1e-4 /
atol 1e-5, as for mhc_pre_clamp_sinkhorn) and against the two operators run
in turn over every token.  Shapes outside the fused kernel (N = 8, fp32,
D % 64 != 0, D < 256) run the two kernels in turn, and the pre forward's
single-pass shapes form x_next inside the single-pass pre kernel; both must
match the two operators bit for bit.  The autograd form must give the
gradients of the unfused chain."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import FlagOS_mhc as m
from test_gpu_post import DEV, _gen, _np, _subset, assert_close, post_inputs
from test_gpu_pre import FWD_KEYS, _oracle_fwd, check_fwd

pytestmark = pytest.mark.gpu

KW = dict(norm_eps=1e-6, hc_eps=1e-6, clamp_min=-10.0, clamp_max=10.0, iter_times=20)


def _inputs(T, N, D, dtype, seed=0):
    x, h_res, h_out, h_post, _ = post_inputs(T, N, D, dtype, seed=seed)
    g = _gen(seed + 100)
    M = 2 * N + N * N
    phi = (torch.randn(M, N * D, device=DEV, generator=g) / (N * D) ** 0.5).to(
        torch.bfloat16 if dtype == torch.bfloat16 else dtype)
    alpha = torch.tensor([0.5, 0.5, 1.0], device=DEV)
    base = torch.randn(M, device=DEV, generator=g) * 0.1
    return x, h_res, h_out, h_post, phi, alpha, base


def _close_gpu(got, want, rtol, atol, what):
    got, want = got.float(), want.float()
    err = (got - want).abs()
    bad = err > atol + rtol * want.abs()
    assert not bool(bad.any()), f"{what}: {int(bad.sum())} / {bad.numel()} outside tol, max err {float(err.max()):.3e}"


def _fused_kernel(T, N, D, dtype):
    """The fused kernel runs for N = 4 bf16, D % 64 == 0 and D >= 256, except
    where the pre forward reads x once (its single pass: T >= 8192, D = 4096
    or 7168 .. 8192 in steps of 256): there the single-pass pre kernel forms
    x_next itself and computes exactly what the two operators compute."""
    single = (N == 4 and dtype == torch.bfloat16 and T >= 8192
              and (D == 4096 or (D % 256 == 0 and 7168 <= D <= 8192)))
    return N == 4 and dtype == torch.bfloat16 and D % 64 == 0 and D >= 256 and not single


CASES = [
    # T, N, D, dtype
    (1000, 4, 4096, torch.bfloat16),    # fused kernel
    (333, 4, 3136, torch.bfloat16),     # fused, partial last 512-column y chunk, ragged tile
    (200, 4, 3584, torch.bfloat16),     # fused
    (4133, 4, 7168, torch.bfloat16),    # fused, D = 7168, several tiles per block
    (31, 4, 7168, torch.bfloat16),      # fused, one partial tile
    (65536, 4, 7168, torch.bfloat16),   # one pass (x_next formed in the single-pass pre kernel), config 5
    (8200, 4, 7168, torch.bfloat16),    # one pass, ragged last tile
    (16390, 4, 4096, torch.bfloat16),   # one pass, two groups per XCC, ragged
    (8192, 4, 6144, torch.bfloat16),    # fused, T in the single-pass range but no slice geometry for D
    (2000, 4, 3072, torch.bfloat16),    # fused
    (77, 4, 256, torch.bfloat16),       # fused, smallest D: a tile spans 4 stages
    (90, 4, 192, torch.bfloat16),       # two kernels: D < 256
    (100, 4, 3600, torch.bfloat16),     # two kernels: D % 64 != 0
    (70, 8, 4096, torch.bfloat16),      # two kernels: N = 8
    (50, 4, 256, torch.float32),        # two kernels: fp32
]


@pytest.mark.parametrize("T,N,D,dtype", CASES)
def test_post_pre_parity(T, N, D, dtype):
    print(f"[post_pre] T={T} N={N} D={D} {dtype} fused={_fused_kernel(T, N, D, dtype)}", flush=True)
    x, h_res, h_out, h_post, phi, alpha, base = _inputs(T, N, D, dtype)
    x_next, out = m.mhc_post_pre_clamp_sinkhorn(x, h_res, h_out, h_post, phi, alpha, base,
                                                need_backward=True, **KW)
    x_ref = m.mhc_post(x, h_res, h_out, h_post)
    ref = m.mhc_pre_clamp_sinkhorn(x_ref, phi, alpha, base, need_backward=True, **KW)
    torch.cuda.synchronize()
    assert x_next.shape == x.shape and x_next.dtype == x.dtype
    assert out["y"].shape == (T, D) and out["x_scaled"] is None
    assert torch.equal(x_next, x_ref), "x_next differs from mhc_post"
    if not _fused_kernel(T, N, D, dtype):
        for k in ("y",) + FWD_KEYS:
            assert torch.equal(out[k], ref[k]), k
        return
    idx = _subset(T)
    want = _oracle_fwd(idx, x_next, phi, alpha, base, KW)
    check_fwd(out, want, dtype, idx, "vs oracle:")
    # every token against the two kernels run in turn (different summation order)
    _close_gpu(out["y"], ref["y"], 2e-2, 2e-2, "y vs unfused")
    for k in FWD_KEYS:
        _close_gpu(out[k], ref[k], 1e-4, 1e-5 + 1e-4 * float(ref[k].abs().max()), k + " vs unfused")
    # deterministic
    x2, out2 = m.mhc_post_pre_clamp_sinkhorn(x, h_res, h_out, h_post, phi, alpha, base,
                                             need_backward=True, **KW)
    assert torch.equal(x2, x_next)
    for k in ("y",) + FWD_KEYS:
        assert torch.equal(out2[k], out[k]), k


def test_post_pre_bsnd_and_no_backward_outputs():
    B, S, N, D = 2, 48, 4, 3584
    x, h_res, h_out, h_post, phi, alpha, base = _inputs(B * S, N, D, torch.bfloat16, seed=3)
    x4 = x.reshape(B, S, N, D)
    x_next, out = m.mhc_post_pre_clamp_sinkhorn(
        x4, h_res.reshape(B, S, N, N), h_out.reshape(B, S, D), h_post.reshape(B, S, N), phi, alpha,
        base, **KW)
    assert x_next.shape == (B, S, N, D) and out["y"].shape == (B, S, D)
    assert set(out) == {"y", "post_out", "comb_frag"}
    x_flat, out_flat = m.mhc_post_pre_clamp_sinkhorn(x, h_res, h_out, h_post, phi, alpha, base, **KW)
    torch.cuda.synchronize()
    assert torch.equal(x_next.reshape(B * S, N, D), x_flat)
    assert torch.equal(out["y"].reshape(B * S, D), out_flat["y"])


@pytest.mark.parametrize("T,D", [(96, 3584), (96, 1024), (1100, 1024), (1100, 5120)])
def test_post_pre_autograd(T, D):
    """x -> fused(post, pre) -> loss on x_next, y, post_out and comb_frag,
    against the unfused autograd chain mhc_post_fn then mhc_pre_clamp_sinkhorn_fn.
    (1100, 1024) takes the accumulating pre backward (the post kernel for
    that shape has no summed form); the others the summed post backward."""
    N = 4
    print(f"[post_pre autograd] T={T} N={N} D={D}", flush=True)
    x, h_res, h_out, h_post, phi, alpha, base = _inputs(T, N, D, torch.bfloat16, seed=7)
    g = _gen(8)
    w_next = torch.randn(T, N, D, device=DEV, generator=g)
    w_y = torch.randn(T, D, device=DEV, generator=g)
    w_p = torch.randn(T, N, device=DEV, generator=g)
    w_c = torch.randn(T, N, N, device=DEV, generator=g)

    def loss(xn, y, p, c):
        return ((xn.float() * w_next).sum() + (y.float() * w_y).sum() + (p * w_p).sum()
                + (c * w_c).sum())

    def leaves():
        return [t.clone().requires_grad_(True) for t in (x, h_res, h_out, h_post, phi, alpha, base)]

    a = leaves()
    loss(*m.mhc_post_pre_clamp_sinkhorn_fn(*a, **KW)).backward()
    b = leaves()
    xn = m.mhc_post_fn(b[0], b[1], b[2], b[3])
    y, p, c = m.mhc_pre_clamp_sinkhorn_fn(xn, b[4], b[5], b[6], **KW)
    loss(xn, y, p, c).backward()
    torch.cuda.synchronize()
    # The fused backward rounds x_next's total gradient at most once (the
    # summed post backward adds grad_x_next and the bf16 dL/dx in fp32; the
    # accumulating pre backward adds them in fp32 and rounds the sum), the
    # unfused chain twice (dL/dx to bf16, then autograd's bf16 add); h_res /
    # h_post gradients are D-long sums over that gradient, so they get an
    # absolute tolerance of 1% of their largest entry.
    for ta, tb, name in zip(a, b, ("x", "h_res", "h_out", "h_post", "phi", "alpha", "base")):
        w = _np(tb.grad)
        atol = (1e-2 if name in ("h_res", "h_post") else 2e-3) * np.abs(w).max()
        assert_close(ta.grad.float(), w, 2e-2, 2e-2 + atol, name + ".grad")


def test_post_pre_one_pass_failure_is_loud():
    """With the waits' limit forced to zero ticks from the host (the
    mhc_debug_set_wait_limit test hook), the one-pass fused forward gives up
    at its first unsatisfied wait and every kernel still exits: x_next, y and
    the pre outputs are NaN, the status word reaches the package, and
    check_errors raises RuntimeError.  With the normal limit restored the
    next call equals the two operators again."""
    from FlagOS_mhc import _lib

    T, N, D = 8192, 4, 7168
    x, h_res, h_out, h_post, phi, alpha, base = _inputs(T, N, D, torch.bfloat16, seed=5)
    lib = _lib.load()
    m.check_errors()  # nothing pending that failed
    try:
        lib.mhc_debug_set_wait_limit(0)
        x_next, out = m.mhc_post_pre_clamp_sinkhorn(x, h_res, h_out, h_post, phi, alpha, base,
                                                    need_backward=True, **KW)
        torch.cuda.synchronize()
        assert bool(torch.isnan(x_next.float()).all()), "x_next"
        for k in ("y",) + FWD_KEYS:
            assert bool(torch.isnan(out[k].float()).all()), k
        with pytest.raises(RuntimeError, match="bounded wait"):
            m.check_errors()
    finally:
        lib.mhc_debug_set_wait_limit(-1)
        torch.cuda.synchronize()
    m.check_errors()
    x_next, out = m.mhc_post_pre_clamp_sinkhorn(x, h_res, h_out, h_post, phi, alpha, base,
                                                need_backward=True, **KW)
    x_ref = m.mhc_post(x, h_res, h_out, h_post)
    ref = m.mhc_pre_clamp_sinkhorn(x_ref, phi, alpha, base, need_backward=True, **KW)
    torch.cuda.synchronize()
    assert torch.equal(x_next, x_ref)
    for k in ("y",) + FWD_KEYS:
        assert torch.equal(out[k], ref[k]), k
    m.check_errors()
