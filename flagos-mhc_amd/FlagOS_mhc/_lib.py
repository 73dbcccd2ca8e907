"""ctypes binding of libmhc_amd.so, the gfx950 HIP kernels behind the ops.

The entry points and their arguments are declared in ``include/mhc_amd.h``.
There is deliberately no fallback: if the library is missing or the tensors
are not on a HIP device, the operators raise instead of computing on the CPU.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

_LIB_NAME = "libmhc_amd.so"
_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), _LIB_NAME)

DTYPE_CODE = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}
PRE_BWD_COMPENSATED = 1  # mhc_pre_bwd_ex flag (include/mhc_amd.h)

_c = ctypes
_vp, _i32, _i64, _f32, _sz = _c.c_void_p, _c.c_int32, _c.c_int64, _c.c_float, _c.c_size_t

_SIGNATURES = {
    "mhc_last_error": (_c.c_char_p, []),
    "mhc_version": (_i32, []),
    "mhc_post_fwd": (_c.c_int, [_vp, _vp, _vp, _vp, _vp, _i64, _i32, _i32, _i32, _vp]),
    "mhc_post_bwd": (_c.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                _i64, _i32, _i32, _i32, _vp]),
    "mhc_post_bwd_sum": (_c.c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                    _i64, _i32, _i32, _i32, _vp]),
    "mhc_post_bwd_sum_fused": (_c.c_int, [_i64, _i32, _i32, _i32]),
    "mhc_pre_fwd_workspace_size": (_sz, [_i64, _i32, _i32, _i32]),
    "mhc_pre_fwd": (_c.c_int, [_vp, _i32, _vp, _i32, _vp, _vp, _f32, _f32, _f32, _f32, _i32,
                               _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz,
                               _i64, _i32, _i32, _vp]),
    "mhc_pre_fwd_noalloc": (_c.c_int, [_vp, _i32, _vp, _i32, _vp, _vp, _f32, _f32, _f32, _f32, _i32,
                                       _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i32, _i32, _vp]),
    "mhc_pre_bwd_acc": (_c.c_int, [_vp, _i32, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                   _f32, _f32, _f32, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _sz,
                                   _i64, _i32, _i32, _vp]),
    "mhc_pre_bwd_ex": (_c.c_int, [_vp, _i32, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                  _f32, _f32, _f32, _i32, _vp, _vp, _vp, _vp, _vp, _c.c_uint32, _vp,
                                  _sz, _i64, _i32, _i32, _vp]),
    "mhc_post_pre_fwd_workspace_size": (_sz, [_i64, _i32, _i32, _i32]),
    "mhc_post_pre_fwd": (_c.c_int, [_vp, _vp, _vp, _vp, _i32, _vp, _i32, _vp, _vp, _f32, _f32, _f32,
                                    _f32, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz,
                                    _i64, _i32, _i32, _vp]),
    "mhc_pre_bwd_workspace_size": (_sz, [_i64, _i32, _i32, _i32, _i32]),
    "mhc_pre_bwd": (_c.c_int, [_vp, _i32, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                               _f32, _f32, _f32, _i32, _vp, _vp, _vp, _vp, _vp, _sz,
                               _i64, _i32, _i32, _vp]),
}

EXPORTED = tuple(_SIGNATURES)

_lock = threading.Lock()
_lib = None


def lib_path() -> str:
    return _LIB_PATH


def load() -> ctypes.CDLL:
    """Load (once) and return the library; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(_LIB_PATH):
                raise RuntimeError(
                    f"{_LIB_NAME} not found at {_LIB_PATH}; build it with "
                    "`python flagos-mhc_amd/build.py` (hipcc, gfx950). The mHC operators "
                    "have no CPU fallback.")
            lib = ctypes.CDLL(_LIB_PATH)
            for name, (res, args) in _SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().mhc_last_error().decode(errors="replace")
        if rc == -2:
            raise NotImplementedError(f"{what}: {msg}")
        raise RuntimeError(f"{what} failed ({rc}): {msg}")


def ptr(t):
    return None if t is None else t.data_ptr()


def stream_of(t: torch.Tensor):
    return torch.cuda.current_stream(t.device).cuda_stream


def require_device(what: str, *tensors) -> None:
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError(
                f"{what}: expected tensors on a HIP (cuda) device, got {t.device}; "
                "the MI355X operators have no CPU path (use the *_ref functions on CPU)")


def dtype_code(what: str, dt: torch.dtype) -> int:
    try:
        return DTYPE_CODE[dt]
    except KeyError:
        raise NotImplementedError(f"{what}: dtype {dt} not supported (float32, bfloat16, float16)")
