"""Argument checks and op registration shared by the Python layer.

`_check` mirrors src/kernels/common.py:6-9: every tensor must live on the GPU,
else ValueError. The reference's `tuned_rows` (common.py:15-34) has no
counterpart: the backward prologue kernel uses a fixed tokens-per-block count.

`custom_op` wraps torch.library.custom_op so that this package never replaces
an op that is already registered. torch.library.custom_op re-binds an existing
name silently, for every caller in the process, and the reference's modules
(src/attention.py, src/kernels/rope.py, ctx_scale.py, fp8.py) register the same
`anima_flat::` names as this package: with both imported, which implementation
ran would depend on import order. Here the second registration raises.
"""

from __future__ import annotations

import torch


def _check(*ts: torch.Tensor) -> None:
    for t in ts:
        if not t.is_cuda:
            raise ValueError("CUDA tensors required")


def is_registered(qualname: str) -> bool:
    """True if the torch.library op `ns::name` exists in this process."""
    ns, name = qualname.split("::", 1)
    return hasattr(getattr(torch.ops, ns), name)


def custom_op(qualname: str, **kwargs):
    """torch.library.custom_op(qualname, **kwargs), refusing an existing name."""
    if is_registered(qualname):
        raise RuntimeError(
            f"torch op {qualname} is already registered in this process (most likely by "
            "anima-flat's own module of the same name); import either that module or "
            "anima_flat_amd's, not both"
        )
    return torch.library.custom_op(qualname, **kwargs)
