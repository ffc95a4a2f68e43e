"""Per-token FP8 quantisation of activations on MI355X.

Drop-in for the `rowquant` part of anima-flat's src/kernels/fp8.py:
`rowquant(x, gelu=False)` (fp8.py:313-328) and the op `anima_flat::rowquant`
(fp8.py:295-310) with the same schema and fake. The Triton kernel
(fp8.py:275-292) is replaced by aa_rowquant. It consumes the attention output
in the model's FP8 path (`rowquant(attention(...))`, model.py:446, 457).

For each token (row of K values): y = x or GELU(x), scale = max(max|y|, 1e-12)
/ 448, q = float8_e4m3fn(clamp(y / scale, -448, 448)) (round to nearest even),
returned as (q [B, S, K], scale [B*S, 1] float32).
"""

from __future__ import annotations

import torch

from .. import _lib
from .common import _check, custom_op

FP8 = torch.float8_e4m3fn
FP8_MAX = 448.0


@custom_op("anima_flat::rowquant", mutates_args=())
def _rowquant(x: torch.Tensor, gelu: bool) -> tuple[torch.Tensor, torch.Tensor]:
    B, S, K = x.shape
    q = torch.empty(B, S, K, dtype=FP8, device=x.device)
    s = torch.empty(B * S, 1, dtype=torch.float32, device=x.device)
    with torch.cuda.device(x.device):
        _lib.check(
            _lib.lib().aa_rowquant(
                x.data_ptr(), B * S, K, int(gelu), q.data_ptr(), s.data_ptr(), _lib.dtype_code(x),
                _lib.stream(x),
            ),
            "rowquant",
        )
    return q, s


@_rowquant.register_fake
def _(x, gelu):
    B, S, K = x.shape
    return (
        torch.empty(B, S, K, dtype=FP8, device=x.device),
        torch.empty(B * S, 1, dtype=torch.float32, device=x.device),
    )


def rowquant(x: torch.Tensor, gelu: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
    """Quantize tokens to FP8 with a scale per token, optionally applying GELU first.

    Args:
        x: Tokens, shape `[B, S, K]`, bfloat16 (K a multiple of 8, at most 8192).
        gelu: Apply GELU before quantizing (the Abramowitz-Stegun erf form, within
            1.5e-7 of the exact erf GELU).

    Returns:
        `(q, s)`: FP8 e4m3fn tokens `[B, S, K]` and their float32 scales `[B * S, 1]`.

    Raises:
        ValueError: If `x` is not on CUDA, or its dtype / K is not supported.
    """
    _check(x)
    return _rowquant(x.contiguous(), gelu)
