"""GPU parity of mhc_pre_clamp_sinkhorn and its backward (HIP kernels via the
C ABI) against the fp64 oracle on token subsets and at small sizes, against
the package's fp32 ``*_ref`` functions run on the GPU at the BASELINE sizes,
and end to end through the autograd wrappers.

Tolerances (north star): fp32 Sinkhorn / mix outputs rtol 1e-4 (atol 1e-5
for entries near zero); bf16 tensors rtol 2e-2 / atol 2e-2 of an fp32 or
better reference; the fp32 T-reductions grad_phi / grad_alpha / grad_base
rtol 1e-4 with atol 1e-5 * max|ref| against a float64 reference over all
tokens (the oracle itself up to 128 tokens, gpu_ref.pre_bwd_fp64 beyond; the
kernels measure a few 1e-6 of max|grad_phi|)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import FlagOS_mhc as m
from gpu_ref import check_reductions, close_gpu, pre_bwd_fp64
from oracle import mhc_oracle as orc
from test_gpu_post import DEV, _gen, _np, _subset, assert_close

pytestmark = pytest.mark.gpu

FWD_KEYS = ("post_out", "comb_frag", "inv_rms", "mixes", "h_res_logits", "pre")


def pre_inputs(T, N, D, dtype=torch.bfloat16, phi_dtype=torch.bfloat16, seed=0, recipe="baseline"):
    g = _gen(seed)
    M = 2 * N + N * N
    if recipe == "baseline":
        x = torch.randn(T, N, D, device=DEV, generator=g).to(dtype)
        phi = (torch.randn(M, N * D, device=DEV, generator=g) / (N * D) ** 0.5).to(phi_dtype)
        alpha = torch.tensor([0.5, 0.5, 1.0], device=DEV)
        base = torch.randn(M, device=DEV, generator=g) * 0.1
    else:                      # reference test recipe (tests/test_correctness.py:74-79)
        x = (torch.randn(T, N, D, device=DEV, generator=g) * 0.1).to(dtype)
        phi = (torch.randn(M, N * D, device=DEV, generator=g) * 0.1).to(phi_dtype)
        alpha = torch.tensor([0.5, 0.5, 0.5], device=DEV)
        base = torch.randn(M, device=DEV, generator=g) * 0.01
    gy = torch.randn(T, D, device=DEV, generator=g).to(dtype)
    gpost = torch.randn(T, N, device=DEV, generator=g)
    gcomb = torch.randn(T, N, N, device=DEV, generator=g)
    return x, phi, alpha, base, gy, gpost, gcomb


def _oracle_fwd(idx, x, phi, alpha, base, kw):
    return orc.pre_fwd(_np(x[idx]), _np(phi), _np(alpha), _np(base), **kw)


def check_fwd(out, want, dtype, idx=None, what=""):
    sel = (lambda t: t[idx]) if idx is not None else (lambda t: t)
    assert_close(sel(out["y"].reshape(-1, out["y"].shape[-1])), want["y"], 2e-2, 2e-2, what + " y")
    for k in FWD_KEYS:
        w = want[k] if isinstance(want[k], np.ndarray) else _np(want[k])
        assert_close(sel(out[k]), w, 1e-4, 1e-5, what + " " + k)


def check_fwd_vs_ref(out, ref, x, phi, alpha, base, kw):
    """Whole outputs against the fp32 torch *_ref.  That reference carries its
    own fp32 rounding (a 16K-deep GEMM), so tokens where the two disagree
    beyond tolerance are settled against the float64 oracle, which both the
    kernel and the tolerance are defined by."""
    T = out["y"].shape[0]
    disputed = np.zeros(T, dtype=bool)
    g, w = _np(out["y"].reshape(T, -1)), _np(ref["y"].reshape(T, -1))
    disputed |= (np.abs(g - w) > 2e-2 + 2e-2 * np.abs(w)).reshape(T, -1).any(1)
    for k in FWD_KEYS:
        g, w = _np(out[k]), _np(ref[k])
        disputed |= (np.abs(g - w) > 1e-5 + 1e-4 * np.abs(w)).reshape(T, -1).any(1)
    idx = np.nonzero(disputed)[0]
    assert idx.size <= max(4, T // 1000), f"{idx.size} of {T} tokens disagree with the fp32 reference"
    if idx.size:
        check_fwd(out, _oracle_fwd(torch.from_numpy(idx).to(DEV), x, phi, alpha, base, kw), None,
                  torch.from_numpy(idx).to(DEV), "oracle (disputed tokens):")


FWD_CASES = [
    # T, N, D, x dtype, phi dtype, recipe, clamp, iters
    (16384, 4, 4096, torch.bfloat16, torch.bfloat16, "baseline", 10.0, 20),   # config 3
    (32768, 8, 2048, torch.bfloat16, torch.bfloat16, "baseline", 10.0, 20),   # config 4
    (16, 4, 64, torch.bfloat16, torch.float32, "reftest", 3.0, 20),           # reference test
    (16, 4, 64, torch.bfloat16, torch.float32, "reftest", 0.0, 20),           # clamp disabled
    (50, 4, 100, torch.bfloat16, torch.bfloat16, "baseline", 10.0, 20),       # D % 8 != 0
    (37, 4, 96, torch.float16, torch.float16, "baseline", 10.0, 7),
    (29, 4, 64, torch.float32, torch.float32, "baseline", 2.0, 20),
    (21, 8, 128, torch.bfloat16, torch.float32, "reftest", 3.0, 1),
    (64, 4, 256, torch.bfloat16, torch.bfloat16, "baseline", 1.0, 0),
    (48, 4, 128, torch.bfloat16, torch.bfloat16, "baseline", 0.5, 45),        # > 32 iterations
    # LDS-pipelined kernel (N=4, bf16): partial last 128-column stages of K and
    # of d, ragged last tile, several tiles per block
    (100, 4, 520, torch.bfloat16, torch.bfloat16, "baseline", 10.0, 20),
    (20000, 4, 1288, torch.bfloat16, torch.bfloat16, "baseline", 10.0, 20),
    (70, 8, 200, torch.bfloat16, torch.bfloat16, "baseline", 10.0, 20),       # N = 8, partial stages
    # N = 8 persistent kernel with the K steps split over waves (more than 256
    # tiles): a partial last stage that ends a short 4-stage MFMA chain, a
    # ragged last tile, blocks with one and two tiles; one stage per tile
    (20000, 8, 200, torch.bfloat16, torch.bfloat16, "baseline", 10.0, 20),
    (16500, 8, 8, torch.bfloat16, torch.bfloat16, "baseline", 10.0, 20),
    # 128-token tiles of 64-column stages (a tile for every CU): ragged last
    # tile, two tiles on the first blocks, one stage per tile
    (33000, 8, 200, torch.bfloat16, torch.bfloat16, "baseline", 10.0, 20),
    (40000, 8, 8, torch.bfloat16, torch.bfloat16, "baseline", 10.0, 20),
    # N=4 bf16 at the model widths D = 1024..8192: ragged last 64-token
    # tiles, fewer tiles than blocks, clamp off, few Sinkhorn iterations
    (1000, 4, 7168, torch.bfloat16, torch.bfloat16, "baseline", 10.0, 20),
    (37, 4, 1024, torch.bfloat16, torch.bfloat16, "baseline", 10.0, 20),
    (700, 4, 2048, torch.bfloat16, torch.bfloat16, "baseline", 3.0, 20),
    (333, 4, 3072, torch.bfloat16, torch.bfloat16, "baseline", 10.0, 5),
    (4133, 4, 5120, torch.bfloat16, torch.bfloat16, "baseline", 10.0, 20),
    (515, 4, 6144, torch.bfloat16, torch.bfloat16, "baseline", 0.0, 20),
    (2050, 4, 8192, torch.bfloat16, torch.bfloat16, "baseline", 10.0, 20),
    (65536, 4, 7168, torch.bfloat16, torch.bfloat16, "baseline", 10.0, 20),  # config 5 (bench)
]


@pytest.mark.parametrize("T,N,D,dtype,phi_dtype,recipe,clamp,iters", FWD_CASES)
def test_pre_fwd_parity(T, N, D, dtype, phi_dtype, recipe, clamp, iters):
    print(f"[pre_fwd] T={T} N={N} D={D} {dtype} phi={phi_dtype} clamp={clamp} it={iters}", flush=True)
    x, phi, alpha, base, *_ = pre_inputs(T, N, D, dtype, phi_dtype, recipe=recipe)
    kw = dict(norm_eps=1e-6, hc_eps=1e-6, clamp_min=-clamp, clamp_max=clamp, iter_times=iters)
    out = m.mhc_pre_clamp_sinkhorn(x, phi, alpha, base, need_backward=True, **kw)
    torch.cuda.synchronize()
    assert out["y"].dtype == dtype and out["y"].shape == (T, D)
    idx = _subset(T)
    want = _oracle_fwd(idx, x, phi, alpha, base, kw)
    check_fwd(out, want, dtype, idx, "oracle:")
    assert_close(out["x_scaled"][idx], want["x_scaled"], 1e-5, 1e-6, "x_scaled")
    if T * N * D >= 1 << 24:   # whole output against the package's fp32 *_ref on the GPU
        ref = m.mhc_pre_clamp_sinkhorn_ref(x, phi, alpha, base, **kw)
        check_fwd_vs_ref(out, ref, x, phi, alpha, base, kw)
    # need_backward=False returns exactly the three outputs, same values
    small = m.mhc_pre_clamp_sinkhorn(x, phi, alpha, base, need_backward=False, **kw)
    assert set(small) == {"y", "post_out", "comb_frag"}
    for k in small:
        assert torch.equal(small[k], out[k])


@pytest.mark.parametrize("T,D", [(4133, 7168), (70, 1024)])
def test_pre_fwd_deterministic(T, D):
    """Every reduction runs in a fixed order (no atomics): two runs give
    identical bits."""
    print(f"[pre_fwd determinism] T={T} D={D}", flush=True)
    x, phi, alpha, base, *_ = pre_inputs(T, 4, D)
    kw = dict(clamp_min=-10.0, clamp_max=10.0)
    a = m.mhc_pre_clamp_sinkhorn(x, phi, alpha, base, need_backward=True, **kw)
    b = m.mhc_pre_clamp_sinkhorn(x, phi, alpha, base, need_backward=True, **kw)
    torch.cuda.synchronize()
    for k in a:
        assert torch.equal(a[k], b[k]), k


def test_pre_fwd_bsnd_shape():
    B, S, N, D = 2, 8, 4, 64
    x, phi, alpha, base, *_ = pre_inputs(B * S, N, D, recipe="reftest", phi_dtype=torch.float32)
    out = m.mhc_pre_clamp_sinkhorn(x.reshape(B, S, N, D), phi, alpha, base, clamp_min=-3.0,
                                   clamp_max=3.0)
    assert out["y"].shape == (B, S, D)
    assert out["post_out"].shape == (B * S, N) and out["comb_frag"].shape == (B * S, N, N)


BWD_CASES = [
    (16384, 4, 4096, torch.bfloat16, torch.bfloat16, "baseline", 10.0, 20),   # config 3 sizes
    (32768, 8, 2048, torch.bfloat16, torch.bfloat16, "baseline", 10.0, 20),   # config 4
    # config-5 width: 56 column blocks x 4 token splits of the grad_x kernel;
    # ragged T with split grad_pre, then the full config 5 (per-token
    # grad_pre in kernel A, byte offsets past 2^31)
    (4133, 4, 7168, torch.bfloat16, torch.bfloat16, "baseline", 10.0, 20),
    (65536, 4, 7168, torch.bfloat16, torch.bfloat16, "baseline", 10.0, 20),   # config 5
    (16, 4, 64, torch.bfloat16, torch.float32, "reftest", 3.0, 20),           # reference test
    (50, 4, 100, torch.bfloat16, torch.bfloat16, "baseline", 0.5, 20),        # D % 8 != 0, clamp active
    (37, 4, 96, torch.float16, torch.float16, "baseline", 10.0, 7),
    (29, 8, 64, torch.float32, torch.float32, "baseline", 2.0, 20),
    (70, 4, 128, torch.bfloat16, torch.bfloat16, "baseline", 0.0, 40),        # scratch Sinkhorn path
    (33, 8, 96, torch.bfloat16, torch.bfloat16, "reftest", 0.2, 1),
    # LDS-pipelined grad_x/grad_phi kernel (N=4, bf16, D % 8 == 0): work ranges
    # that cross column blocks, a partial last column block, a ragged last tile
    (1010, 4, 1288, torch.bfloat16, torch.bfloat16, "baseline", 10.0, 20),
    # more column blocks than CUs (several waves of blocks)
    (17, 4, 40000, torch.bfloat16, torch.bfloat16, "baseline", 10.0, 20),
    # few column blocks: many more token splits of the grad_phi partials
    (4000, 4, 256, torch.bfloat16, torch.bfloat16, "baseline", 10.0, 20),
    # grad_pre: bf16 rows with 16-byte alignment at T >= 16384 (N = 4 and 8)
    # take the LDS-pipelined pre_bwd_gpre_dma_kernel (70001 x 8 x 64); N = 4
    # in other dtypes at T >= 16384 a wave per token in kernel A; everything
    # else the split (token, 2048-column) partials of pre_bwd_gpre_kernel,
    # whose grid holds at most 65536 token blocks, so at 70001 tokens with
    # unaligned rows (D = 60) its blocks loop over several tokens
    (3, 4, 7168, torch.bfloat16, torch.bfloat16, "baseline", 10.0, 20),
    (4, 8, 100, torch.float32, torch.float32, "baseline", 10.0, 20),
    (5, 4, 4100, torch.float16, torch.float16, "baseline", 10.0, 20),
    (70001, 8, 64, torch.bfloat16, torch.bfloat16, "baseline", 10.0, 20),
    (70001, 8, 60, torch.bfloat16, torch.bfloat16, "baseline", 10.0, 20),
    # N = 8 grad_x kernel with two waves per stream (64-column halves): a
    # last column block whose second half is partly past D, a ragged last tile
    (1000, 8, 1000, torch.bfloat16, torch.bfloat16, "baseline", 10.0, 20),
]


@pytest.mark.parametrize("T,N,D,dtype,phi_dtype,recipe,clamp,iters", BWD_CASES)
def test_pre_bwd_parity(T, N, D, dtype, phi_dtype, recipe, clamp, iters):
    print(f"[pre_bwd] T={T} N={N} D={D} {dtype} phi={phi_dtype} clamp={clamp} it={iters}", flush=True)
    x, phi, alpha, base, gy, gpost, gcomb = pre_inputs(T, N, D, dtype, phi_dtype, recipe=recipe)
    kw = dict(norm_eps=1e-6, hc_eps=1e-6, clamp_min=-clamp, clamp_max=clamp, iter_times=iters)
    out = m.mhc_pre_clamp_sinkhorn(x, phi, alpha, base, need_backward=True, **kw)
    gx, gphi, ga, gb = m.mhc_pre_clamp_sinkhorn_backward(
        x, phi, alpha, base, out["inv_rms"], out["x_scaled"], out["mixes"], out["h_res_logits"],
        out["pre"], gy, gpost, gcomb, **kw)
    torch.cuda.synchronize()
    assert gx.dtype == dtype and gx.shape == x.shape
    assert gphi.dtype == torch.float32 and gphi.shape == phi.shape
    if T <= 128:
        want = orc.pre_bwd(_np(x), _np(phi), _np(alpha), _np(base), _np(gy), _np(gpost),
                           _np(gcomb), **kw)
        assert_close(gx, want[0], 2e-2, 2e-2, "grad_x")
        for got, w, name in ((gphi, want[1], "grad_phi"), (ga, want[2], "grad_alpha"),
                             (gb, want[3], "grad_base")):
            assert_close(got, w, 1e-4, 1e-5 * np.abs(w).max(), name)
    else:
        # per-token grad_x against the oracle on a subset, every token and the
        # T-reductions against the float64 reference
        idx = _subset(T)
        sub = orc.pre_bwd(_np(x[idx]), _np(phi), _np(alpha), _np(base), _np(gy[idx]),
                          _np(gpost[idx]), _np(gcomb[idx]), **kw)
        assert_close(gx[idx], sub[0], 2e-2, 2e-2, "grad_x subset vs oracle")
        ref = pre_bwd_fp64(x, phi, alpha, base, gy, gpost, gcomb, kw, grad_x=gx)
        check_reductions(gphi, ga, gb, ref)
    # deterministic: no atomics anywhere
    again = m.mhc_pre_clamp_sinkhorn_backward(
        x, phi, alpha, base, out["inv_rms"], None, out["mixes"], None, out["pre"], gy, gpost,
        gcomb, **kw)
    for a, b in zip(again, (gx, gphi, ga, gb)):
        assert torch.equal(a, b)


@pytest.mark.parametrize("T,N,D,dtype", [
    (1000, 4, 1024, torch.bfloat16),    # LDS-pipelined kernel, grad_x_in accumulated in place
    (4133, 4, 7168, torch.bfloat16),
    (70, 8, 256, torch.bfloat16),       # LDS-pipelined kernel, two stream groups, grad_x_in in place
    (40, 4, 100, torch.bfloat16),       # D % 8 != 0: generic kernel + separate add
    (33, 4, 64, torch.float32),
])
def test_pre_bwd_accumulate(T, N, D, dtype):
    """mhc_pre_bwd_acc: grad_x = grad_x_in + dL/dx (one rounding), the other
    gradients bit-identical to mhc_pre_bwd."""
    from FlagOS_mhc.mhc_pre_clamp_sinkhorn_backward import _pre_backward
    print(f"[pre_bwd acc] T={T} N={N} D={D} {dtype}", flush=True)
    x, phi, alpha, base, gy, gpost, gcomb = pre_inputs(T, N, D, dtype, dtype if dtype != torch.bfloat16 else torch.bfloat16)
    kw = dict(norm_eps=1e-6, hc_eps=1e-6, clamp_min=-10.0, clamp_max=10.0, iter_times=20)
    out = m.mhc_pre_clamp_sinkhorn(x, phi, alpha, base, need_backward=True, **kw)
    gin = torch.randn(x.shape, device=DEV, generator=_gen(9)).to(dtype)
    args = (x, phi, alpha, base, out["inv_rms"], out["mixes"], out["pre"], gy, gpost, gcomb,
            kw["norm_eps"], kw["hc_eps"], kw["clamp_min"], kw["clamp_max"], kw["iter_times"])
    gx, gphi, ga, gb = _pre_backward(*args)
    gxa, gphia, gaa, gba = _pre_backward(*args, grad_x_in=gin)
    torch.cuda.synchronize()
    assert gxa.shape == x.shape and gxa.dtype == dtype
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    assert_close(gxa.float(), (gx.float() + gin.float()), tol, tol, "grad_x_in + grad_x")
    for a, b, name in ((gphia, gphi, "phi"), (gaa, ga, "alpha"), (gba, gb, "base")):
        assert torch.equal(a, b), name


def _comp_inputs(T, N, D, dtype, recipe, seed=0):
    """recipe "pos": x ~ 1 + 0.25 N(0,1) and grad_y = |N(0,1)|, so grad_pre and
    with it the grad_mixes of the pre head keep one sign over all tokens and
    grad_phi's T-sums grow without cancelling; "rand": the baseline recipe."""
    x, phi, alpha, base, gy, gpost, gcomb = pre_inputs(T, N, D, dtype, dtype, seed=seed)
    if recipe == "pos":
        g = _gen(seed + 50)
        x = (1 + 0.25 * torch.randn(T, N, D, device=DEV, generator=g)).to(dtype)
        gy = torch.randn(T, D, device=DEV, generator=g).abs().to(dtype)
    return x, phi, alpha, base, gy, gpost, gcomb


COMP_CASES = [
    # T, N, D, dtype, recipe -- kernel path of the rest of the backward
    (8192, 4, 64, torch.bfloat16, "pos"),    # LDS-pipelined grad_x kernel
    (8192, 4, 64, torch.bfloat16, "rand"),
    (4096, 8, 96, torch.bfloat16, "pos"),    # register-streaming kernel (N = 8)
    (3000, 4, 100, torch.float16, "pos"),    # LDS-staged kernel, D % 8 != 0 (element-wise x loads)
    (2000, 4, 64, torch.float32, "pos"),     # three x planes
    (1500, 8, 40, torch.float32, "pos"),
    (37, 4, 64, torch.bfloat16, "rand"),     # one partial 32-token tile
    (1, 4, 64, torch.bfloat16, "pos"),
]


@pytest.mark.parametrize("T,N,D,dtype,recipe", COMP_CASES)
def test_pre_bwd_compensated(T, N, D, dtype, recipe):
    """compensated=True (mhc_pre_bwd_ex, MHC_PRE_BWD_COMPENSATED): grad_phi,
    grad_alpha and grad_base against the float64 oracle over every token.
    Measured on MI355X, the default path's grad_phi is 3e-7 .. 4e-6 of
    max|grad_phi| off the oracle on these cases (fp32 recursive sums, g in two
    bf16 planes), the compensated one 7e-8 .. 1.6e-7 (the fp32 grad_mixes
    themselves); the bound 3e-7 fails the default path on most cases.  grad_x
    is the default path's, bit for bit; results repeat bit for bit."""
    print(f"[pre_bwd compensated] T={T} N={N} D={D} {dtype} {recipe}", flush=True)
    x, phi, alpha, base, gy, gpost, gcomb = _comp_inputs(T, N, D, dtype, recipe)
    kw = dict(norm_eps=1e-6, hc_eps=1e-6, clamp_min=-10.0, clamp_max=10.0, iter_times=20)
    out = m.mhc_pre_clamp_sinkhorn(x, phi, alpha, base, need_backward=True, **kw)
    args = (x, phi, alpha, base, out["inv_rms"], None, out["mixes"], None, out["pre"], gy, gpost, gcomb)
    plain = m.mhc_pre_clamp_sinkhorn_backward(*args, **kw)
    comp = m.mhc_pre_clamp_sinkhorn_backward(*args, **kw, compensated=True)
    again = m.mhc_pre_clamp_sinkhorn_backward(*args, **kw, compensated=True)
    torch.cuda.synchronize()
    for a, b in zip(comp, again):
        assert torch.equal(a, b)
    assert torch.equal(comp[0], plain[0]), "grad_x must not change"
    want = orc.pre_bwd(_np(x), _np(phi), _np(alpha), _np(base), _np(gy), _np(gpost), _np(gcomb), **kw)

    def rel(got, w):
        return float(np.abs(_np(got).astype(np.float64) - w).max() / np.abs(w).max())

    e_comp, e_plain = rel(comp[1], want[1]), rel(plain[1], want[1])
    print(f"  grad_phi max error / max: default {e_plain:.2e}, compensated {e_comp:.2e}", flush=True)
    assert e_comp <= 3e-7, e_comp
    if T >= 8192 and recipe == "pos":
        assert e_comp * 4 <= e_plain, (e_comp, e_plain)
    for got, w, name in ((comp[2], want[2], "grad_alpha"), (comp[3], want[3], "grad_base")):
        assert rel(got, w) <= 1e-6, name


def test_pre_bwd_compensated_c5_width():
    """D = 7168 (K = 28672: 224 column blocks, several token splits): the
    compensated grad_phi agrees with the default path's to its accuracy, and
    the autograd wrapper forwards the option."""
    T, N, D = 4133, 4, 7168
    print(f"[pre_bwd compensated] T={T} N={N} D={D}", flush=True)
    x, phi, alpha, base, gy, gpost, gcomb = pre_inputs(T, N, D)
    kw = dict(norm_eps=1e-6, hc_eps=1e-6, clamp_min=-10.0, clamp_max=10.0, iter_times=20)
    out = m.mhc_pre_clamp_sinkhorn(x, phi, alpha, base, need_backward=True, **kw)
    args = (x, phi, alpha, base, out["inv_rms"], None, out["mixes"], None, out["pre"], gy, gpost, gcomb)
    plain = m.mhc_pre_clamp_sinkhorn_backward(*args, **kw)
    comp = m.mhc_pre_clamp_sinkhorn_backward(*args, **kw, compensated=True)
    torch.cuda.synchronize()
    assert torch.equal(comp[0], plain[0])
    for a, b, name in zip(comp[1:], plain[1:], ("grad_phi", "grad_alpha", "grad_base")):
        assert_close(a, _np(b), 1e-4, 2e-5 * float(b.abs().max()), name)
    leaves = [t.clone().requires_grad_(True) for t in (x, phi, alpha, base)]
    y, p, c = m.mhc_pre_clamp_sinkhorn_fn(*leaves, **kw, compensated=True)
    ((y.float() * gy.float()).sum() + (p * gpost).sum() + (c * gcomb).sum()).backward()
    torch.cuda.synchronize()
    assert torch.equal(leaves[1].grad.float(), comp[1].to(phi.dtype).float())
    assert torch.equal(leaves[2].grad, comp[2]) and torch.equal(leaves[3].grad, comp[3])


def test_pre_bwd_empty_batch():
    N, D = 4, 64
    x, phi, alpha, base, *_ = pre_inputs(1, N, D)
    e = lambda *s: torch.empty(*s, device=DEV)
    gx, gphi, ga, gb = m.mhc_pre_clamp_sinkhorn_backward(
        x[:0], phi, alpha, base, e(0), None, e(0, 24), None, e(0, N),
        torch.empty(0, D, dtype=x.dtype, device=DEV), e(0, N), e(0, N, N))
    torch.cuda.synchronize()
    assert gx.shape == (0, N, D)
    assert not gphi.any() and not ga.any() and not gb.any()


@pytest.mark.parametrize("N", [4, 8])
def test_autograd_chain(N):
    """pre -> h_out = y + noise -> post -> loss, through the autograd wrappers,
    against the same chain through the package's *_ref functions in fp32."""
    T, D = 96, 128
    x, phi, alpha, base, *_ = pre_inputs(T, N, D, recipe="baseline")
    g = _gen(5)
    noise = (torch.randn(T, D, device=DEV, generator=g) * 0.1).to(x.dtype)
    upstream = torch.randn(T, N, D, device=DEV, generator=g).to(x.dtype)
    kw = dict(norm_eps=1e-6, hc_eps=1e-6, clamp_min=-10.0, clamp_max=10.0, iter_times=20)

    leaves = [t.clone().requires_grad_(True) for t in (x, phi, alpha, base)]
    y, post, comb = m.mhc_pre_clamp_sinkhorn_fn(*leaves, **kw)
    out = m.mhc_post_fn(leaves[0], comb, y + noise, post)
    (out.float() * upstream.float()).sum().backward()

    rl = [t.detach().float().requires_grad_(True) for t in (x, phi, alpha, base)]
    r = m.mhc_pre_clamp_sinkhorn_ref(*rl, **kw)
    r_out = m.mhc_post_ref(rl[0], r["comb_frag"], r["y"] + noise.float(), r["post_out"])
    (r_out * upstream.float()).sum().backward()

    assert_close(out, r_out, 2e-2, 2e-2, "chain output")
    assert_close(leaves[0].grad, rl[0].grad, 2e-2, 2e-2, "x.grad")
    for a, b, name in ((leaves[1], rl[1], "phi"), (leaves[2], rl[2], "alpha"), (leaves[3], rl[3], "base")):
        w = _np(b.grad)
        assert_close(a.grad.float(), w, 2e-2, 2e-3 * np.abs(w).max(), name + ".grad")


@pytest.mark.parametrize("N,D", [(4, 7168), (4, 100), (8, 2048)])
def test_pre_bwd_clamp_bounds_inclusive(N, D):
    """F7 on the GPU: with phi = 0 the logits equal base exactly, and some sit
    exactly on +-clamp.  The kernel's clamp gradient must pass there, as
    torch.clamp's does for the reference's *_ref (src/mhc_pre_clamp_sinkhorn_
    backward.py:1434-1435; its Triton path is strict, :1186-1191): grad_base
    against the oracle, non-zero on the bounds and zero outside them."""
    from test_ref import clamp_bound_base
    T, c = 300, 0.5
    M = 2 * N + N * N
    print(f"[pre_bwd clamp bounds] T={T} N={N} D={D}", flush=True)
    x, _, alpha, _, gy, gpost, gcomb = pre_inputs(T, N, D)
    phi = torch.zeros(M, N * D, device=DEV, dtype=torch.bfloat16)
    base = torch.from_numpy(clamp_bound_base(N, c, np.random.default_rng(N + D))).to(DEV)
    kw = dict(norm_eps=1e-6, hc_eps=1e-6, clamp_min=-c, clamp_max=c, iter_times=20)
    out = m.mhc_pre_clamp_sinkhorn(x, phi, alpha, base, need_backward=True, **kw)
    lg = base[2 * N:].reshape(N, N)
    assert torch.equal(out["h_res_logits"], lg.expand(T, N, N))   # logits == base, bit for bit
    gx, gphi, ga, gb = m.mhc_pre_clamp_sinkhorn_backward(
        x, phi, alpha, base, out["inv_rms"], None, out["mixes"], None, out["pre"], gy, gpost, gcomb, **kw)
    torch.cuda.synchronize()
    want = orc.pre_bwd(_np(x), _np(phi), _np(alpha), _np(base), _np(gy), _np(gpost), _np(gcomb), **kw)
    assert_close(gb, want[3], 1e-4, 1e-5 * np.abs(want[3]).max(), "grad_base")
    # the logit block at its own scale (the pre head's sums dominate max|grad_base|)
    gl, wl = _np(gb)[2 * N:].reshape(N, N), want[3][2 * N:].reshape(N, N)
    assert_close(gl, wl, 1e-4, 1e-5 * np.abs(wl).max(), "grad_base logit block")
    lgn = _np(lg)
    assert (gl[np.abs(lgn) == c] != 0).all(), "gradient must pass on the bounds (a strict mask gives 0)"
    assert (gl[np.abs(lgn) > c] == 0).all(), "no gradient outside the clamp range"
    assert_close(gx, want[0], 2e-2, 2e-2, "grad_x")
    assert_close(gphi, want[1], 1e-4, 1e-5 * np.abs(want[1]).max(), "grad_phi")


def test_autograd_chain_config5():
    """BASELINE config 5 end to end at its size (N=4, D=7168, T=65536, bf16,
    clamp +-10, 20 iterations), as the reference's harness runs its chain
    (tests/test_correctness.py:98-142): mhc_pre_clamp_sinkhorn_fn -> h_out =
    y + N(0, 0.1) noise -> mhc_post_fn -> backward of an N(0,1) upstream
    gradient through both autograd Functions.
      * x.grad on a token subset against the float64 oracle chain (bf16 tol);
      * phi / alpha / base grads against the fp32 *_ref autograd chain on the
        GPU over all tokens (rtol 2e-2, atol 2e-3 * max: the two chains store
        different intermediates, bf16 y and grad_h_out here, fp32 there);
      * and, tightly, the fp32 grad_phi / grad_alpha / grad_base of the same
        gradients against the float64 pre backward (rtol 1e-4, atol 1e-5 *
        max); the wrapper's grads equal them (phi.grad cast to phi's dtype)."""
    T, N, D = 65536, 4, 7168
    print(f"[chain config 5] T={T} N={N} D={D}", flush=True)
    x, phi, alpha, base, *_ = pre_inputs(T, N, D, recipe="baseline")
    g = _gen(5)
    noise = (torch.randn(T, D, device=DEV, generator=g) * 0.1).to(x.dtype)
    upstream = torch.randn(T, N, D, device=DEV, generator=g).to(x.dtype)
    kw = dict(norm_eps=1e-6, hc_eps=1e-6, clamp_min=-10.0, clamp_max=10.0, iter_times=20)

    leaves = [t.clone().requires_grad_(True) for t in (x, phi, alpha, base)]
    y, post, comb = m.mhc_pre_clamp_sinkhorn_fn(*leaves, **kw)
    h_out = y + noise
    out = m.mhc_post_fn(leaves[0], comb, h_out, post)
    out.backward(upstream)
    torch.cuda.synchronize()
    print("  HIP chain done", flush=True)

    # x.grad per token: oracle chain on a subset (post backward at the chain's
    # own gates and h_out, then the pre backward of its gradients)
    idx = _subset(T)
    f = lambda t: _np(t[idx])
    ofwd = orc.pre_fwd(f(x), _np(phi), _np(alpha), _np(base), **kw)
    assert_close(comb[idx], ofwd["comb_frag"], 1e-4, 1e-5, "comb_frag")
    assert_close(post[idx], ofwd["post_out"], 1e-4, 1e-5, "post_out")
    assert_close(out[idx], orc.post_fwd(f(x), f(comb), f(h_out), f(post)), 2e-2, 2e-2, "chain output")
    gpx, ghr, gho, ghp = orc.post_bwd(f(upstream), f(x), f(comb), f(h_out), f(post))
    gprx = orc.pre_bwd(f(x), _np(phi), _np(alpha), _np(base), gho, ghp, ghr, **kw)[0]
    assert_close(leaves[0].grad[idx], gpx + gprx, 3e-2, 3e-2, "x.grad subset vs oracle chain")

    # T-reductions, tightly.  The wrapper returns grad_phi in phi's dtype
    # (bf16 here), as the reference's does; it must equal the fp32 result of
    # a direct call on the gradients the chain's post backward produced (all
    # kernels are deterministic, so they are recomputed here), and that fp32
    # result is held to the float64 pre backward of the same gradients.
    pb = m.mhc_post_backward(upstream, x, comb.detach(), h_out.detach(), post.detach())
    fo = m.mhc_pre_clamp_sinkhorn(x, phi, alpha, base, need_backward=True, **kw)
    gd = m.mhc_pre_clamp_sinkhorn_backward(x, phi, alpha, base, fo["inv_rms"], None, fo["mixes"], None,
                                           fo["pre"], pb[2], pb[3], pb[1], **kw)
    assert leaves[1].grad.dtype == phi.dtype
    assert torch.equal(leaves[1].grad, gd[1].to(phi.dtype)), "phi.grad"
    assert torch.equal(leaves[2].grad, gd[2]) and torch.equal(leaves[3].grad, gd[3]), "alpha / base .grad"
    assert torch.equal(leaves[0].grad, pb[0] + gd[0]), "x.grad = post + pre contributions"
    ref = pre_bwd_fp64(x, phi, alpha, base, pb[2], pb[3], pb[1], kw)
    check_reductions(gd[1], gd[2], gd[3], ref, "chain vs fp64")
    del pb, fo, gd, ref
    print("  fp64 reductions ok", flush=True)

    # the fp32 *_ref chain over all tokens
    rl = [t.detach().float().requires_grad_(True) for t in (x, phi, alpha, base)]
    r = m.mhc_pre_clamp_sinkhorn_ref(*rl, **kw)
    r_out = m.mhc_post_ref(rl[0], r["comb_frag"], r["y"] + noise.float(), r["post_out"])
    r_out.backward(upstream.float())
    torch.cuda.synchronize()
    close_gpu(out, r_out, 2e-2, 2e-2, "chain output vs fp32 *_ref")
    del r_out, r
    close_gpu(leaves[0].grad, rl[0].grad, 3e-2, 3e-2, "x.grad vs fp32 *_ref")
    for a, b, name in ((leaves[1], rl[1], "phi"), (leaves[2], rl[2], "alpha"), (leaves[3], rl[3], "base")):
        close_gpu(a.grad.float(), b.grad, 2e-2, 2e-3 * float(b.grad.abs().max()), name + ".grad vs fp32 *_ref")
