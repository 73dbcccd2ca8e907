"""Writes the golden fixtures of this directory from the CPU oracle.

The reference ships no golden vectors (its only test compares two live
computations at T=16, tests/test_correctness.py:25-32), so these fixtures are
produced by oracle/mhc_oracle.py -- itself pinned by closed forms, brute force
and finite differences (tests/test_oracle.py).  They freeze seeded inputs and
expected outputs so that GPU parity tests and oracle changes are checked
against fixed data.

Inputs are stored as float32 arrays holding bf16-representable values (for
the bf16 cases) so they convert to bf16 exactly; expected outputs are float64
oracle results stored as float64.

Usage:  python tests/golden/make_golden.py      (rewrites mhc_golden.npz)
"""

from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import mhc_oracle as orc  # noqa: E402


def bf16(a):
    a32 = np.asarray(a, dtype=np.float32)
    u = a32.view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16 << 16
    return u.astype(np.uint32).view(np.float32)


POST_CASES = [
    # name, T, N, D, gate recipe
    ("post_ref_test", 16, 4, 64, "randn"),      # reference harness shapes (B=2, S=8)
    ("post_softmax_n8", 24, 8, 40, "softmax"),
    ("post_n2_odd", 9, 2, 13, "randn"),
]

PRE_CASES = [
    # name, T, N, D, recipe, clamp, iters
    ("pre_ref_test", 16, 4, 64, "reftest", 3.0, 20),   # tests/test_correctness.py:74-115
    ("pre_baseline_n4", 20, 4, 48, "baseline", 10.0, 20),
    ("pre_noclamp_n8", 12, 8, 32, "baseline", 0.0, 20),
    ("pre_iter1_n4", 8, 4, 24, "reftest", 0.5, 1),
    ("pre_iter40_n4", 8, 4, 16, "baseline", 0.2, 40),
]


def main():
    r = np.random.default_rng(20261201)
    out = {}
    for name, T, N, D, gates in POST_CASES:
        x = bf16(r.standard_normal((T, N, D)))
        h_out = bf16(r.standard_normal((T, D)))
        if gates == "softmax":
            z = r.standard_normal((T, N, N))
            h_res = (np.exp(z) / np.exp(z).sum(-1, keepdims=True)).astype(np.float32)
            h_post = (r.random((T, N)) * 2).astype(np.float32)
        else:
            h_res = r.standard_normal((T, N, N)).astype(np.float32)
            h_post = r.standard_normal((T, N)).astype(np.float32)
        gy = bf16(r.standard_normal((T, N, D)))
        y = orc.post_fwd(x, h_res, h_out, h_post)
        gx, ghr, gho, ghp = orc.post_bwd(gy, x, h_res, h_out, h_post)
        for k, v in dict(x=x, h_res=h_res, h_out=h_out, h_post=h_post, grad_y=gy, y=y,
                         grad_x=gx, grad_h_res=ghr, grad_h_out=gho, grad_h_post=ghp).items():
            out[f"{name}/{k}"] = v
    for name, T, N, D, recipe, clamp, iters in PRE_CASES:
        M = 2 * N + N * N
        if recipe == "reftest":
            x = bf16(r.standard_normal((T, N, D)) * 0.1)
            phi = (r.standard_normal((M, N * D)) * 0.1).astype(np.float32)
            alpha = np.array([0.5, 0.5, 0.5], np.float32)
            base = (r.standard_normal(M) * 0.01).astype(np.float32)
        else:
            x = bf16(r.standard_normal((T, N, D)))
            phi = bf16(r.standard_normal((M, N * D)) / np.sqrt(N * D))
            alpha = np.array([0.5, 0.5, 1.0], np.float32)
            base = (r.standard_normal(M) * 0.1).astype(np.float32)
        gy = bf16(r.standard_normal((T, D)))
        gpost = r.standard_normal((T, N)).astype(np.float32)
        gcomb = r.standard_normal((T, N, N)).astype(np.float32)
        kw = dict(norm_eps=1e-6, hc_eps=1e-6, clamp_min=-clamp, clamp_max=clamp, iter_times=iters)
        fwd = orc.pre_fwd(x, phi, alpha, base, **kw)
        gx, gphi, ga, gb = orc.pre_bwd(x, phi, alpha, base, gy, gpost, gcomb, **kw)
        arrays = dict(x=x, phi=phi, alpha=alpha, base=base, grad_y=gy, grad_post_out=gpost,
                      grad_comb_frag=gcomb, grad_x=gx, grad_phi=gphi, grad_alpha=ga, grad_base=gb,
                      hyper=np.array([1e-6, 1e-6, -clamp, clamp, iters], np.float64))
        arrays.update({f"fwd_{k}": v for k, v in fwd.items()})
        for k, v in arrays.items():
            out[f"{name}/{k}"] = v
    path = os.path.join(HERE, "mhc_golden.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path}: {len(out)} arrays, {os.path.getsize(path)} bytes")


if __name__ == "__main__":
    main()
