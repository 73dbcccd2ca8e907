"""mhc_pre_fwd_noalloc, the allocation-free pre forward (its workspace is a
static per-GPU device array), against mhc_pre_fwd with a caller workspace,
both called through the C ABI.  Pairs of calls in a row, the second smaller,
so the second runs on scratch left over from the first; every output must be
bit-identical to mhc_pre_fwd's (same kernels)."""

from __future__ import annotations

import pytest
import torch

from FlagOS_mhc import _lib

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs(T, N, D, phi_dtype, seed):
    g = torch.Generator(device=DEV)
    g.manual_seed(seed)
    M = 2 * N + N * N
    x = torch.randn(T, N, D, device=DEV, generator=g).to(torch.bfloat16)
    phi = (torch.randn(M, N * D, device=DEV, generator=g) / (N * D) ** 0.5).to(phi_dtype)
    alpha = torch.tensor([0.5, 0.5, 1.0], device=DEV)
    base = torch.randn(M, device=DEV, generator=g) * 0.1
    return x, phi, alpha, base


def _run(noalloc, x, phi, alpha, base, clamp=10.0, iters=20):
    T, N, D = x.shape
    M = 2 * N + N * N
    f32 = dict(device=DEV, dtype=torch.float32)
    o = {"y": torch.empty(T, D, device=DEV, dtype=x.dtype), "post_out": torch.empty(T, N, **f32),
         "comb_frag": torch.empty(T, N, N, **f32), "inv_rms": torch.empty(T, **f32),
         "mixes": torch.empty(T, M, **f32), "h_res_logits": torch.empty(T, N, N, **f32),
         "pre": torch.empty(T, N, **f32), "x_scaled": torch.empty(T, N * D, **f32)}
    lib = _lib.load()
    xc, pc = _lib.DTYPE_CODE[x.dtype], _lib.DTYPE_CODE[phi.dtype]
    head = (x.data_ptr(), xc, phi.data_ptr(), pc, alpha.data_ptr(), base.data_ptr(), 1e-6, 1e-6,
            -clamp, clamp, iters) + tuple(o[k].data_ptr() for k in o)
    stream = torch.cuda.current_stream().cuda_stream
    if noalloc:
        rc = lib.mhc_pre_fwd_noalloc(*head, T, N, D, stream)
    else:
        ws = torch.empty(max(1, lib.mhc_pre_fwd_workspace_size(T, N, D, pc)), dtype=torch.uint8, device=DEV)
        rc = lib.mhc_pre_fwd(*head, ws.data_ptr(), ws.numel(), T, N, D, stream)
    _lib.check(rc, "noalloc" if noalloc else "mhc_pre_fwd")
    return o


PAIRS = [
    # (T, N, D, phi dtype) first call, then a smaller T: persistent kernel, split-K kernels
    ((20000, 4, 1024, torch.bfloat16), 300),
    ((4133, 4, 7168, torch.bfloat16), 100),
    ((3000, 8, 2048, torch.bfloat16), 64),       # N = 8: tile sums + finalize kernel
    ((33000, 8, 200, torch.bfloat16), 20000),    # N = 8 persistent K-split kernel: 128-, then 64-token tiles
    ((500, 4, 520, torch.float32), 37),          # fp32 phi split into bf16 planes in the scratch
]


@pytest.mark.parametrize("first,t2", PAIRS, ids=[f"T{p[0][0]}-N{p[0][1]}-D{p[0][2]}" for p in PAIRS])
def test_noalloc_matches_workspace_entry(first, t2):
    T, N, D, pdt = first
    for step, t in enumerate((T, t2)):
        print(f"[pre_fwd_noalloc] call {step + 1}: T={t} N={N} D={D} phi={pdt}", flush=True)
        x, phi, alpha, base = _inputs(t, N, D, pdt, seed=11 * step + N)
        got = _run(True, x, phi, alpha, base)
        want = _run(False, x, phi, alpha, base)
        torch.cuda.synchronize()
        for k in want:
            assert torch.equal(got[k], want[k]), (step, k)


def test_noalloc_refuses_above_its_scratch():
    lib = _lib.load()
    T = 5_000_000   # N = 4: 20 B of workspace per token, above the 64 MiB scratch
    assert lib.mhc_pre_fwd_workspace_size(T, 4, 1024, 1) > 64 << 20
    x = torch.empty(1, device=DEV)
    p = x.data_ptr()
    rc = lib.mhc_pre_fwd_noalloc(p, 1, p, 1, p, p, 1e-6, 1e-6, 0.0, 0.0, 20, p, p, p, None, None, None,
                                 None, None, T, 4, 1024, torch.cuda.current_stream().cuda_stream)
    assert rc == -1 and b"static scratch" in lib.mhc_last_error()
