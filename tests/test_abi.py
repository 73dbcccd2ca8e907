"""C-ABI checks that need no GPU: the library loads, exports every entry
point declared in include/mhc_amd.h, rejects bad arguments with the right
codes before touching the device, and the Python operators refuse CPU
tensors instead of falling back."""

from __future__ import annotations

import ctypes
import os
import re

import pytest
import torch

from conftest import PKG_DIR, ROOT

HEADER = os.path.join(ROOT, "include", "mhc_amd.h")


@pytest.fixture(scope="module")
def lib():
    from FlagOS_mhc import _lib
    if not os.path.exists(_lib.lib_path()):
        import importlib.util
        spec = importlib.util.spec_from_file_location("mhc_build", os.path.join(PKG_DIR, "build.py"))
        mod = importlib.util.module_from_spec(spec)
        spec.loader.exec_module(mod)
        mod.build()
    return _lib.load()


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mhc_[a-z0-9_]+)\s*\(", text)))


def test_header_matches_binding():
    from FlagOS_mhc import _lib
    assert sorted(_lib.EXPORTED) == _declared()


def test_library_exports_every_declared_symbol(lib):
    for name in _declared():
        assert hasattr(lib, name), name
    path = lib._name
    raw = ctypes.CDLL(path)
    for name in _declared():
        assert ctypes.cast(getattr(raw, name), ctypes.c_void_p).value


def test_version_and_error_string(lib):
    assert lib.mhc_version() >= 100
    assert isinstance(lib.mhc_last_error(), bytes)


def test_workspace_sizes(lib):
    # bf16 phi is used in place: the workspace holds pre (T,N) and inv_rms (T,) for the y kernel
    assert lib.mhc_pre_fwd_workspace_size(65536, 4, 5120, 1) == 256 + 65536 * 4 * 4 + 65536 * 4
    # D = 7168: also room for the single-pass form (control words, exchange
    # ring, the [T][24] and [T] sums for the finalize kernel, then pre / inv_rms)
    assert lib.mhc_pre_fwd_workspace_size(65536, 4, 7168, 1) > 256 + 65536 * (16 + 4 + 25 * 4)
    fp32 = lib.mhc_pre_fwd_workspace_size(65536, 4, 7168, 0)
    assert fp32 >= 2 * 24 * 28672 * 2
    ws20 = lib.mhc_pre_bwd_workspace_size(65536, 4, 7168, 1, 20)
    ws40 = lib.mhc_pre_bwd_workspace_size(65536, 4, 7168, 1, 40)
    assert ws20 >= 65536 * 24 * 4 and ws40 > ws20
    assert lib.mhc_pre_bwd_workspace_size(0, 4, 7168, 1, 20) > 0


def test_error_codes_without_device(lib):
    dummy = ctypes.c_void_p(0x1000)
    # unsupported N is rejected before any launch
    rc = lib.mhc_post_fwd(dummy, dummy, dummy, dummy, dummy, 16, 3, 64, 1, None)
    assert rc == -2 and b"N=3" in lib.mhc_last_error()
    rc = lib.mhc_post_fwd(None, dummy, dummy, dummy, dummy, 16, 4, 64, 1, None)
    assert rc == -1 and b"null" in lib.mhc_last_error()
    rc = lib.mhc_post_fwd(dummy, dummy, dummy, dummy, dummy, 16, 4, 64, 7, None)
    assert rc == -2
    rc = lib.mhc_pre_fwd(dummy, 1, dummy, 1, dummy, dummy, 1e-6, 1e-6, 0.0, 0.0, 20,
                         dummy, dummy, dummy, None, None, None, None, None, None, 0,
                         16, 6, 64, None)
    assert rc == -2
    rc = lib.mhc_pre_bwd(dummy, 1, dummy, 1, dummy, dummy, dummy, dummy, dummy, dummy, dummy,
                         dummy, 1e-6, 0.0, 0.0, 20, dummy, dummy, dummy, dummy, dummy, 16,
                         16, 4, 64, None)
    assert rc == -1 and b"workspace" in lib.mhc_last_error()
    # token counts beyond 32-bit grids are refused, not wrapped
    big = 1 << 32
    rc = lib.mhc_post_fwd(dummy, dummy, dummy, dummy, dummy, big, 4, 64, 1, None)
    assert rc == -2 and b"above the supported" in lib.mhc_last_error()
    rc = lib.mhc_post_bwd(dummy, dummy, dummy, dummy, dummy, dummy, dummy, dummy, dummy, big, 4, 64, 1, None)
    assert rc == -2 and b"above the supported" in lib.mhc_last_error()
    rc = lib.mhc_pre_fwd(dummy, 1, dummy, 1, dummy, dummy, 1e-6, 1e-6, 0.0, 0.0, 20,
                         dummy, dummy, dummy, None, None, None, None, None, dummy, 1 << 20, big, 4, 64, None)
    assert rc == -2 and b"above the supported" in lib.mhc_last_error()
    rc = lib.mhc_pre_bwd(dummy, 1, dummy, 1, dummy, dummy, dummy, dummy, dummy, dummy, dummy,
                         dummy, 1e-6, 0.0, 0.0, 20, dummy, dummy, dummy, dummy, dummy, 16, big, 4, 64, None)
    assert rc == -2 and b"above the supported" in lib.mhc_last_error()
    # T == 0 is a no-op for the forward ops
    assert lib.mhc_post_fwd(dummy, dummy, dummy, dummy, dummy, 0, 4, 64, 1, None) == 0
    # accumulating pre backward: grad_x_in is required and must not overlap grad_x
    gx, gin_ok, gin_overlap = ctypes.c_void_p(0x100000), ctypes.c_void_p(0x900000), ctypes.c_void_p(0x100400)
    acc = lambda gin, out: lib.mhc_pre_bwd_acc(
        dummy, 1, dummy, 1, dummy, dummy, dummy, dummy, dummy, dummy, dummy, dummy, 1e-6, 0.0, 0.0, 20,
        gin, out, dummy, dummy, dummy, dummy, 16, 16, 4, 64, None)
    assert acc(None, gx) == -1 and b"null grad_x_in" in lib.mhc_last_error()
    assert acc(gx, gx) == -1 and b"overlaps" in lib.mhc_last_error()
    assert acc(gin_overlap, gx) == -1 and b"overlaps" in lib.mhc_last_error()   # 16*4*64*2 bytes
    assert acc(gin_ok, gx) == -1 and b"workspace" in lib.mhc_last_error()       # passes to mhc_pre_bwd's checks
    # pre backward with options: unknown flag bits, overlap, then mhc_pre_bwd's checks
    ex = lambda gin, flags: lib.mhc_pre_bwd_ex(
        dummy, 1, dummy, 1, dummy, dummy, dummy, dummy, dummy, dummy, dummy, dummy, 1e-6, 0.0, 0.0, 20,
        gin, gx, dummy, dummy, dummy, flags, None, dummy, 16, 16, 4, 64, None)
    assert ex(None, 8) == -1 and b"flags" in lib.mhc_last_error()
    assert ex(None, 6) == -1 and b"together" in lib.mhc_last_error()   # both pass flags
    assert ex(None, 2) == -1 and b"workspace" in lib.mhc_last_error()  # MHC_PRE_BWD_TWO_PASS is known
    assert ex(None, 4) == -1 and b"workspace" in lib.mhc_last_error()  # MHC_PRE_BWD_SINGLE_PASS is known
    assert ex(gin_overlap, 1) == -1 and b"overlaps" in lib.mhc_last_error()
    assert ex(None, 1) == -1 and b"workspace" in lib.mhc_last_error()
    assert ex(gin_ok, 0) == -1 and b"workspace" in lib.mhc_last_error()
    # fused post + pre forward: N outside {4, 8} and null pointers are rejected before any launch
    fused = lambda x, n: lib.mhc_post_pre_fwd(
        x, dummy, dummy, dummy, 1, dummy, 1, dummy, dummy, 1e-6, 1e-6, 0.0, 0.0, 20, dummy, dummy, dummy,
        dummy, None, None, None, None, dummy, 256, 16, n, 64, None)
    assert fused(dummy, 6) == -2 and b"N=6" in lib.mhc_last_error()
    assert fused(None, 4) == -1 and b"null" in lib.mhc_last_error()


def test_ops_refuse_cpu_tensors():
    import FlagOS_mhc as m
    x = torch.zeros(16, 4, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="HIP"):
        m.mhc_post(x, torch.zeros(16, 4, 4), torch.zeros(16, 64, dtype=torch.bfloat16),
                   torch.zeros(16, 4))
    phi = torch.zeros(24, 256)
    with pytest.raises(RuntimeError, match="HIP"):
        m.mhc_pre_clamp_sinkhorn(x, phi, torch.zeros(3), torch.zeros(24))


def test_public_api_names():
    """The reference's twelve names (src/__init__.py:34-47) come first and
    unchanged; the additions are the fused post+pre operator, the post
    backward for a gradient given as two summands and the single-pass
    forward's failure check."""
    import FlagOS_mhc as m
    assert m.__all__[:12] == [
        "mhc_post", "mhc_post_ref", "mhc_post_backward", "mhc_post_backward_ref",
        "mhc_pre_clamp_sinkhorn", "mhc_pre_clamp_sinkhorn_ref",
        "mhc_pre_clamp_sinkhorn_backward", "mhc_pre_clamp_sinkhorn_backward_ref",
        "MhcPostFn", "MhcPreClampSinkhornFn", "mhc_post_fn", "mhc_pre_clamp_sinkhorn_fn",
    ]
    assert m.__all__[12:] == [
        "mhc_post_pre_clamp_sinkhorn", "MhcPostPreClampSinkhornFn", "mhc_post_pre_clamp_sinkhorn_fn",
        "mhc_post_backward_sum", "check_errors",
    ]
    for name in m.__all__:
        assert callable(getattr(m, name))


def test_noalloc_pre_fwd_refuses_sizes_above_its_scratch(lib):
    """mhc_pre_fwd_noalloc checks the workspace it would need against its
    static scratch before touching the device."""
    T = 5_000_000
    assert lib.mhc_pre_fwd_workspace_size(T, 4, 1024, 1) > 64 << 20
    rc = lib.mhc_pre_fwd_noalloc(None, 1, None, 1, None, None, 1e-6, 1e-6, 0.0, 0.0, 20, None, None,
                                 None, None, None, None, None, None, T, 4, 1024, None)
    assert rc == -1 and b"static scratch" in lib.mhc_last_error()
    assert lib.mhc_pre_fwd_noalloc(None, 1, None, 1, None, None, 1e-6, 1e-6, 0.0, 0.0, 20, None, None,
                                   None, None, None, None, None, None, -1, 4, 1024, None) == -1
