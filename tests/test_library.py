"""torch.library registration of the mHC operators (FlagOS_mhc.library).

CPU: the six ops are registered, their shape functions give the real
kernels' output shapes / dtypes on meta tensors, and the real implementations
refuse CPU tensors (no CPU path).  GPU: torch.library.opcheck (schema,
fake-tensor and autograd registration checks), compiled mHC layers (unfused
and fused post + pre; torch.compile, aot_eager backend, fullgraph) against
the same layers run eagerly through the autograd wrappers, and HIP-graph
capture of the four-op
chain replayed several times against eager results (bit equality: the kernels
are deterministic and the replay runs the same launches)."""

from __future__ import annotations

import pytest
import torch

import FlagOS_mhc as m
from FlagOS_mhc import library as L

OPS = ("mhc_post", "mhc_post_backward", "mhc_pre_clamp_sinkhorn", "mhc_pre_clamp_sinkhorn_backward",
       "mhc_pre_clamp_sinkhorn_backward_acc", "mhc_post_pre_clamp_sinkhorn")


def test_ops_registered():
    for name in OPS:
        assert hasattr(torch.ops.flagos_mhc, name), name


@pytest.mark.parametrize("lead", [(6,), (2, 3)])
@pytest.mark.parametrize("N", [4, 8])
def test_meta_shapes(lead, N):
    D, M = 16, N * (N + 2)
    T = 6
    with torch.device("meta"):
        x = torch.empty(lead + (N, D), dtype=torch.bfloat16)
        h_res = torch.empty(lead + (N, N))
        h_out = torch.empty(lead + (D,), dtype=torch.bfloat16)
        h_post = torch.empty(lead + (N,))
        phi = torch.empty(M, N * D, dtype=torch.bfloat16)
        alpha, base = torch.empty(3), torch.empty(M)
        y = torch.ops.flagos_mhc.mhc_post(x, h_res, h_out, h_post)
        assert y.shape == x.shape and y.dtype == x.dtype
        gx, ghr, gho, ghp = torch.ops.flagos_mhc.mhc_post_backward(x, x, h_res, h_out, h_post)
        assert (gx.shape, gx.dtype) == (x.shape, x.dtype)
        assert (ghr.shape, ghr.dtype) == (h_res.shape, torch.float32)
        assert (gho.shape, gho.dtype) == (lead + (D,), torch.bfloat16)
        assert (ghp.shape, ghp.dtype) == (h_post.shape, torch.float32)
        outs = torch.ops.flagos_mhc.mhc_pre_clamp_sinkhorn(x, phi, alpha, base, 1e-6, 1e-6, 0.0, 0.0, 20)
        want = [(lead + (D,), torch.bfloat16), ((T, N), torch.float32), ((T, N, N), torch.float32),
                ((T,), torch.float32), ((T, M), torch.float32), ((T, N), torch.float32)]
        assert [(tuple(o.shape), o.dtype) for o in outs] == want
        y, post_out, comb, inv, mixes, pre = outs
        g = torch.ops.flagos_mhc.mhc_pre_clamp_sinkhorn_backward(
            x, phi, alpha, base, inv, mixes, pre, y, post_out, comb, 1e-6, 1e-6, 0.0, 0.0, 20)
        assert [(tuple(o.shape), o.dtype) for o in g] == [
            (x.shape, torch.bfloat16), ((M, N * D), torch.float32), ((3,), torch.float32),
            ((M,), torch.float32)]
        f = torch.ops.flagos_mhc.mhc_post_pre_clamp_sinkhorn(x, h_res, h_out, h_post, phi, alpha, base,
                                                             1e-6, 1e-6, 0.0, 0.0, 20)
        assert [(tuple(o.shape), o.dtype) for o in f] == [(x.shape, torch.bfloat16)] + want


def test_cpu_tensors_refused():
    x = torch.randn(4, 4, 8)
    with pytest.raises(RuntimeError, match="HIP"):
        torch.ops.flagos_mhc.mhc_post(x, torch.randn(4, 4, 4), torch.randn(4, 8), torch.randn(4, 4))


# ---- GPU ---------------------------------------------------------------------

DEV = "cuda"
KW = dict(norm_eps=1e-6, hc_eps=1e-6, clamp_min=-10.0, clamp_max=10.0, iter_times=20)


def _layer_inputs(T, N, D, seed=0):
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    M = N * (N + 2)
    x = torch.randn(T, N, D, device=DEV, generator=g).to(torch.bfloat16)
    phi = (torch.randn(M, N * D, device=DEV, generator=g) / (N * D) ** 0.5).to(torch.bfloat16)
    alpha = torch.tensor([0.5, 0.5, 1.0], device=DEV)
    base = torch.randn(M, device=DEV, generator=g) * 0.1
    noise = (torch.randn(T, D, device=DEV, generator=g) * 0.1).to(torch.bfloat16)
    upstream = torch.randn(T, N, D, device=DEV, generator=g).to(torch.bfloat16)
    return x, phi, alpha, base, noise, upstream


@pytest.mark.gpu
def test_opcheck():
    T, N, D = 40, 4, 64
    print(f"[opcheck] T={T} N={N} D={D}", flush=True)
    x, phi, alpha, base, noise, upstream = _layer_inputs(T, N, D)
    g = torch.Generator(device=DEV)
    g.manual_seed(3)
    h_res = torch.softmax(torch.randn(T, N, N, device=DEV, generator=g), -1)
    h_post = torch.rand(T, N, device=DEV, generator=g) * 2
    args = tuple(KW.values())
    torch.library.opcheck(torch.ops.flagos_mhc.mhc_post.default,
                          (x.requires_grad_(True), h_res, noise, h_post))
    torch.library.opcheck(torch.ops.flagos_mhc.mhc_post_backward.default,
                          (upstream, x.detach(), h_res, noise, h_post))
    leaves = (x.detach().requires_grad_(True), phi.requires_grad_(True), alpha, base)
    torch.library.opcheck(torch.ops.flagos_mhc.mhc_pre_clamp_sinkhorn.default, leaves + args)
    y, post_out, comb, inv, mixes, pre = torch.ops.flagos_mhc.mhc_pre_clamp_sinkhorn(
        x.detach(), phi.detach(), alpha, base, *args)
    bwd_args = (x.detach(), phi.detach(), alpha, base, inv, mixes, pre, noise,
                torch.randn_like(post_out), torch.randn_like(comb)) + args
    torch.library.opcheck(torch.ops.flagos_mhc.mhc_pre_clamp_sinkhorn_backward.default, bwd_args)
    # the compensated reductions (trailing bool) through the same ops
    torch.library.opcheck(torch.ops.flagos_mhc.mhc_pre_clamp_sinkhorn_backward.default, bwd_args + (True,))
    torch.library.opcheck(torch.ops.flagos_mhc.mhc_pre_clamp_sinkhorn.default, leaves + args + (True,))


@pytest.mark.gpu
def test_registered_op_compensated_gradients():
    """compensated=True through the registered op's autograd gives the
    functional compensated backward's gradients, bit for bit."""
    T, N, D = 300, 4, 512
    print(f"[op compensated] T={T} N={N} D={D}", flush=True)
    x, phi, alpha, base, noise, _ = _layer_inputs(T, N, D, seed=5)
    g = torch.Generator(device=DEV)
    g.manual_seed(6)
    gpost = torch.randn(T, N, device=DEV, generator=g)
    gcomb = torch.randn(T, N, N, device=DEV, generator=g)
    leaves = [t.clone().requires_grad_(True) for t in (x, phi, alpha, base)]
    y, p, c = L.mhc_pre_clamp_sinkhorn_op(*leaves, **KW, compensated=True)
    ((y.float() * noise.float()).sum() + (p * gpost).sum() + (c * gcomb).sum()).backward()
    out = m.mhc_pre_clamp_sinkhorn(x, phi, alpha, base, need_backward=True, **KW)
    gx, gphi, ga, gb = m.mhc_pre_clamp_sinkhorn_backward(
        x, phi, alpha, base, out["inv_rms"], None, out["mixes"], None, out["pre"], noise, gpost, gcomb,
        **KW, compensated=True)
    torch.cuda.synchronize()
    assert torch.equal(leaves[0].grad, gx)
    assert torch.equal(leaves[1].grad, gphi.to(phi.dtype))
    assert torch.equal(leaves[2].grad, ga) and torch.equal(leaves[3].grad, gb)


@pytest.mark.gpu
def test_opcheck_post_pre():
    T, N, D = 40, 4, 3136   # the fused kernel (D >= 256, D % 64 == 0)
    print(f"[opcheck post_pre] T={T} N={N} D={D}", flush=True)
    x, phi, alpha, base, noise, upstream = _layer_inputs(T, N, D)
    g = torch.Generator(device=DEV)
    g.manual_seed(4)
    h_res = torch.softmax(torch.randn(T, N, N, device=DEV, generator=g), -1)
    h_post = torch.rand(T, N, device=DEV, generator=g) * 2
    torch.library.opcheck(torch.ops.flagos_mhc.mhc_post_pre_clamp_sinkhorn.default,
                          (x.requires_grad_(True), h_res, noise, h_post, phi.requires_grad_(True), alpha,
                           base) + tuple(KW.values()))


@pytest.mark.gpu
def test_compiled_fused_layer_matches_eager():
    """x -> fused(post, pre) op -> loss, compiled (aot_eager, fullgraph) and
    eager through the autograd Function."""
    T, N, D = 64, 4, 3136
    print(f"[compile post_pre] T={T} N={N} D={D}", flush=True)
    x, phi, alpha, base, noise, upstream = _layer_inputs(T, N, D, seed=21)
    g = torch.Generator(device=DEV)
    g.manual_seed(22)
    h_res = torch.softmax(torch.randn(T, N, N, device=DEV, generator=g), -1)
    h_post = torch.rand(T, N, device=DEV, generator=g) * 2
    w = torch.randn(T, D, device=DEV, generator=g)

    def loss_of(fn, *a):
        xn, y, p, c = fn(*a, **KW)
        return (xn.float() * upstream.float()).sum() + (y.float() * w).sum() + p.sum() + c.sum()

    def run(fn):
        leaves = [t.clone().requires_grad_(True) for t in (x, h_res, noise, h_post, phi, alpha, base)]
        loss_of(fn, *leaves).backward()
        return [t.grad for t in leaves]

    torch._dynamo.reset()
    compiled = torch.compile(lambda *a: loss_of(L.mhc_post_pre_clamp_sinkhorn_op, *a), backend="aot_eager",
                             fullgraph=True)

    def run_compiled():
        leaves = [t.clone().requires_grad_(True) for t in (x, h_res, noise, h_post, phi, alpha, base)]
        compiled(*leaves).backward()
        return [t.grad for t in leaves]

    got = run_compiled()
    want = run(m.mhc_post_pre_clamp_sinkhorn_fn)
    torch.cuda.synchronize()
    for a, b, name in zip(got, want, ("x", "h_res", "h_out", "h_post", "phi", "alpha", "base")):
        torch.testing.assert_close(a.float(), b.float(), rtol=1e-5, atol=1e-5, msg=name)


def _layer(ops, x, phi, alpha, base, noise, upstream):
    if ops:
        y, post, comb = L.mhc_pre_clamp_sinkhorn_op(x, phi, alpha, base, **KW)
        out = L.mhc_post_op(x, comb, y + noise, post)
    else:
        y, post, comb = m.mhc_pre_clamp_sinkhorn_fn(x, phi, alpha, base, **KW)
        out = m.mhc_post_fn(x, comb, y + noise, post)
    return (out.float() * upstream.float()).sum(), out


@pytest.mark.gpu
@pytest.mark.parametrize("N", [4, 8])
def test_compiled_layer_matches_eager(N):
    T, D = 96, 128
    print(f"[compile aot_eager] T={T} N={N} D={D}", flush=True)
    x, phi, alpha, base, noise, upstream = _layer_inputs(T, N, D, seed=N)

    def run(fn):
        leaves = [t.clone().requires_grad_(True) for t in (x, phi, alpha, base)]
        loss, out = fn(*leaves, noise, upstream)
        loss.backward()
        return [out.detach()] + [t.grad for t in leaves]

    torch._dynamo.reset()
    compiled = torch.compile(lambda *a: _layer(True, *a), backend="aot_eager", fullgraph=True)
    got = run(compiled)
    want = run(lambda *a: _layer(False, *a))
    torch.cuda.synchronize()
    for a, b, name in zip(got, want, ("out", "x", "phi", "alpha", "base")):
        assert a.shape == b.shape and a.dtype == b.dtype, name
        torch.testing.assert_close(a.float(), b.float(), rtol=1e-5, atol=1e-5, msg=name)


def _chain(x, phi, alpha, base, noise, upstream, gpost, gcomb):
    """Forward and backward of pre and post through the registered ops
    (explicit backward calls, no autograd): every output of the four ops."""
    args = tuple(KW.values())
    y, post_out, comb, inv, mixes, pre = torch.ops.flagos_mhc.mhc_pre_clamp_sinkhorn(
        x, phi, alpha, base, *args)
    out = torch.ops.flagos_mhc.mhc_post(x, comb, noise, post_out)
    gx, ghr, gho, ghp = torch.ops.flagos_mhc.mhc_post_backward(upstream, x, comb, noise, post_out)
    gx2, gphi, ga, gb = torch.ops.flagos_mhc.mhc_pre_clamp_sinkhorn_backward(
        x, phi, alpha, base, inv, mixes, pre, gho, gpost, gcomb, *args)
    return [y, post_out, comb, inv, mixes, pre, out, gx, ghr, gho, ghp, gx2, gphi, ga, gb]


@pytest.mark.gpu
@pytest.mark.parametrize("T,N,D", [(300, 4, 512), (130, 8, 256)])
def test_hip_graph_replay(T, N, D):
    print(f"[hip graph] T={T} N={N} D={D}", flush=True)
    x, phi, alpha, base, noise, upstream = _layer_inputs(T, N, D, seed=11)
    g = torch.Generator(device=DEV)
    g.manual_seed(12)
    gpost = torch.randn(T, N, device=DEV, generator=g)
    gcomb = torch.randn(T, N, N, device=DEV, generator=g)
    static = [x, phi, alpha, base, noise, upstream, gpost, gcomb]

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        _chain(*static)  # warm-up outside capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = _chain(*static)
    torch.cuda.synchronize()

    for rnd in range(4):
        if rnd == 2:  # new input contents: the replay must read them
            g.manual_seed(13)
            x.copy_(torch.randn(T, N, D, device=DEV, generator=g).to(x.dtype))
            upstream.copy_(torch.randn(T, N, D, device=DEV, generator=g).to(upstream.dtype))
        eager = _chain(*static)  # eager work between the replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(captured, eager)):
            assert torch.equal(a, b), f"replay {rnd}: output {i} differs from eager"
