"""MI355X (gfx950) implementation of the four mHC operators.

Drop-in for the reference package's public API (src/__init__.py:34-47): the
same twelve names, signatures and return conventions.  The operators run
hand-written HIP kernels from ``libmhc_amd.so`` (built by
``flagos-mhc_amd/build.py``) on the current HIP stream; the ``*_ref``
functions are the pure-PyTorch references of the same semantics.

    mhc_post                       (forward)
    mhc_post_backward
    mhc_pre_clamp_sinkhorn         (forward, returns dict)
    mhc_pre_clamp_sinkhorn_backward
    mhc_post_fn, mhc_pre_clamp_sinkhorn_fn   (autograd wrappers)

Beyond the reference: ``mhc_post_pre_clamp_sinkhorn`` (and its autograd
form) fuses mhc_post of one layer with mhc_pre_clamp_sinkhorn of the next;
``mhc_post_backward_sum`` is mhc_post_backward for a gradient given as two
summands (the fused layer's backward); ``check_errors`` raises if an earlier
single-pass pre forward gave up one of its bounded waits (the pre backward
and every later pre forward check that too).

Importing the package also registers the operators as torch.ops.flagos_mhc.*
(``FlagOS_mhc.library``) for torch.compile and HIP-graph capture.
"""

from .mhc_post import mhc_post, mhc_post_ref
from .mhc_post_backward import mhc_post_backward, mhc_post_backward_ref, mhc_post_backward_sum
from .mhc_pre_clamp_sinkhorn import (
    mhc_pre_clamp_sinkhorn,
    mhc_pre_clamp_sinkhorn_ref,
)
from .mhc_pre_clamp_sinkhorn_backward import (
    mhc_pre_clamp_sinkhorn_backward,
    mhc_pre_clamp_sinkhorn_backward_ref,
)
from .autograd import (
    MhcPostFn,
    MhcPreClampSinkhornFn,
    mhc_post_fn,
    mhc_pre_clamp_sinkhorn_fn,
    MhcPostPreClampSinkhornFn,
    mhc_post_pre_clamp_sinkhorn_fn,
)
from .mhc_post_pre import mhc_post_pre_clamp_sinkhorn
from ._lib import check_errors
from . import library  # registers torch.ops.flagos_mhc.* (torch.compile / HIP graphs)

__all__ = [
    "mhc_post",
    "mhc_post_ref",
    "mhc_post_backward",
    "mhc_post_backward_ref",
    "mhc_pre_clamp_sinkhorn",
    "mhc_pre_clamp_sinkhorn_ref",
    "mhc_pre_clamp_sinkhorn_backward",
    "mhc_pre_clamp_sinkhorn_backward_ref",
    "MhcPostFn",
    "MhcPreClampSinkhornFn",
    "mhc_post_fn",
    "mhc_pre_clamp_sinkhorn_fn",
    # beyond the reference: mhc_post (layer l) fused with mhc_pre_clamp_sinkhorn (layer l+1)
    "mhc_post_pre_clamp_sinkhorn",
    "MhcPostPreClampSinkhornFn",
    "mhc_post_pre_clamp_sinkhorn_fn",
    # beyond the reference: mhc_post_backward for a gradient given as two summands
    "mhc_post_backward_sum",
    # beyond the reference: reports a single-pass pre forward that gave up a bounded wait
    "check_errors",
]
