"""Argument checks shared by the prologue and padding-correction ops.

Mirrors src/kernels/common.py:6-9 (`_check`): every tensor must live on the
GPU, else ValueError. The reference's `tuned_rows` (common.py:15-34) has no
counterpart: the backward prologue kernel uses a fixed tokens-per-block count.
"""

from __future__ import annotations

import torch


def _check(*ts: torch.Tensor) -> None:
    for t in ts:
        if not t.is_cuda:
            raise ValueError("CUDA tensors required")
