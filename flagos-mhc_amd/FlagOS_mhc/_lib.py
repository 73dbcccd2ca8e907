"""ctypes binding of libmhc_amd.so, the gfx950 HIP kernels behind the ops.

The entry points and their arguments are declared in ``include/mhc_amd.h``.
There is deliberately no fallback: if the library is missing or the tensors
are not on a HIP device, the operators raise instead of computing on the CPU.
"""

from __future__ import annotations

import collections
import ctypes
import os
import threading

import torch

_LIB_NAME = "libmhc_amd.so"
_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), _LIB_NAME)

DTYPE_CODE = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}
PRE_BWD_COMPENSATED = 1  # mhc_pre_bwd_ex flags (include/mhc_amd.h)
PRE_BWD_TWO_PASS = 2
PRE_BWD_SINGLE_PASS = 4

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
    "mhc_pre_fwd_ex": (_c.c_int, [_vp, _i32, _vp, _i32, _vp, _vp, _f32, _f32, _f32, _f32, _i32,
                                  _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp,
                                  _i64, _i32, _i32, _vp]),
    "mhc_debug_set_wait_limit": (None, [_i64]),
    "mhc_pre_fwd_noalloc": (_c.c_int, [_vp, _i32, _vp, _i32, _vp, _vp, _f32, _f32, _f32, _f32, _i32,
                                       _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i32, _i32, _vp]),
    "mhc_pre_bwd_acc": (_c.c_int, [_vp, _i32, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                   _f32, _f32, _f32, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _sz,
                                   _i64, _i32, _i32, _vp]),
    "mhc_pre_bwd_ex": (_c.c_int, [_vp, _i32, _vp, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                  _f32, _f32, _f32, _i32, _vp, _vp, _vp, _vp, _vp, _c.c_uint32, _vp,
                                  _vp, _sz, _i64, _i32, _i32, _vp]),
    "mhc_post_pre_fwd_workspace_size": (_sz, [_i64, _i32, _i32, _i32]),
    "mhc_post_pre_fwd": (_c.c_int, [_vp, _vp, _vp, _vp, _i32, _vp, _i32, _vp, _vp, _f32, _f32, _f32,
                                    _f32, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz,
                                    _i64, _i32, _i32, _vp]),
    "mhc_post_pre_fwd_ex": (_c.c_int, [_vp, _vp, _vp, _vp, _i32, _vp, _i32, _vp, _vp, _f32, _f32, _f32,
                                       _f32, _i32, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp,
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


class SinglePassStatus:
    """Where the single-pass pre forward and backward report their bounded waits.

    Those kernels wait for the other CUs of their group with a limit (0.25 s
    without progress); if a wait gives up, the call's outputs are NaN and the
    kernels write a failure code to the status word of ``mhc_pre_fwd_ex`` /
    ``mhc_pre_bwd_ex``.
    Each call gets a word in a ring of pinned host memory (written by the GPU
    with a system-scope store, read by the host once the call's event has
    completed), so no call waits for the GPU.  ``check`` raises for a failed
    call: without blocking at the start of every operator call (calls whose
    work has finished), blocking in the pre backward and in
    ``FlagOS_mhc.check_errors``."""

    # enough that a caller enqueueing far ahead of the GPU never waits for a
    # word (16 KB of pinned memory)
    SLOTS = 4096

    def __init__(self):
        self._lock = threading.RLock()
        self._words = None
        self._busy = [False] * self.SLOTS
        self._next = 0
        self._pending = collections.deque()  # (slot, event), oldest first

    def acquire(self):
        """A zeroed word for the next call: (slot, its address).  A word is
        reused only after the call that reported into it was checked."""
        with self._lock:
            if self._words is None:
                self._words = torch.zeros(self.SLOTS, dtype=torch.int32, pin_memory=True)
            while self._busy[self._next]:
                self.check(block=True)
            slot = self._next
            self._next = (slot + 1) % self.SLOTS
            self._words[slot] = 0
            return slot, self._words.data_ptr() + 4 * slot

    def commit(self, slot, stream) -> None:
        """The call that got `slot` was enqueued on `stream`."""
        ev = torch.cuda.Event()
        ev.record(stream)
        with self._lock:
            self._busy[slot] = True
            self._pending.append((slot, ev))

    def check(self, block: bool) -> None:
        if torch.cuda.is_available() and torch.cuda.is_current_stream_capturing():
            return
        with self._lock:
            while self._pending:
                slot, ev = self._pending[0]
                if not block and not ev.query():
                    return
                ev.synchronize()
                self._pending.popleft()
                self._busy[slot] = False
                code = int(self._words[slot])
                if code:
                    raise RuntimeError(
                        f"mhc_pre_clamp_sinkhorn: an earlier single-pass forward or backward call gave "
                        f"up a bounded wait for the other CUs of its group (status {code}: the GPU "
                        "stalled longer than the wait limit); that call's outputs are NaN")


SINGLE_PASS = SinglePassStatus()


def check_errors(block: bool = True) -> None:
    """Raise RuntimeError if an earlier single-pass pre forward or backward
    gave up a bounded wait (its outputs are then NaN).  With ``block`` (the default)
    wait for every such call's work to finish first; without it, look only
    at calls that have finished."""
    SINGLE_PASS.check(block)
