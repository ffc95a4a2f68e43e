"""Padding correction of trimmed cross-attention on MI355X.

Drop-in for anima-flat's src/kernels/ctx_scale.py: `ctx_scale(out, lse,
ln_pad)` (ctx_scale.py:141-147) and the ops `anima_flat::ctx_scale` /
`anima_flat::ctx_scale_bwd` with the same schemas, fakes and autograd. The
Triton kernels are replaced by aa_ctx_scale_fwd / aa_ctx_scale_bwd.

y = out * g, g = 1 / (1 + exp(ln_pad[b] - lse[b, h, s])): attention over the
first len keys, times g, equals attention over the context zero-padded to
S_full keys when ln_pad = log(S_full - len).
"""

from __future__ import annotations

import torch

from .. import _lib
from .common import _check, custom_op


def _check_hd(hd: int) -> None:
    if hd != 128:
        raise ValueError(f"head_dim {hd} is not supported (128 only)")


@custom_op("anima_flat::ctx_scale", mutates_args=())
def _ctx_scale(out: torch.Tensor, lse: torch.Tensor, ln_pad: torch.Tensor) -> torch.Tensor:
    B, S, H, hd = out.shape
    _check_hd(hd)
    y = torch.empty_like(out)
    with torch.cuda.device(out.device):
        _lib.check(
            _lib.lib().aa_ctx_scale_fwd(
                out.data_ptr(),
                lse.data_ptr(),
                ln_pad.data_ptr(),
                y.data_ptr(),
                B,
                S,
                H,
                hd,
                _lib.dtype_code(out),
                _lib.stream(out),
            ),
            "ctx_scale",
        )
    return y


@_ctx_scale.register_fake
def _(out, lse, ln_pad):
    return torch.empty_like(out)


@custom_op("anima_flat::ctx_scale_bwd", mutates_args=())
def _ctx_scale_bwd_op(
    out: torch.Tensor, lse: torch.Tensor, ln_pad: torch.Tensor, dy: torch.Tensor
) -> tuple[torch.Tensor, torch.Tensor]:
    B, S, H, hd = out.shape
    _check_hd(hd)
    dy = dy.contiguous()
    dout = torch.empty_like(out)
    dlse = torch.empty_like(lse)
    with torch.cuda.device(out.device):
        _lib.check(
            _lib.lib().aa_ctx_scale_bwd(
                out.data_ptr(),
                lse.data_ptr(),
                ln_pad.data_ptr(),
                dy.data_ptr(),
                dout.data_ptr(),
                dlse.data_ptr(),
                B,
                S,
                H,
                hd,
                _lib.dtype_code(out),
                _lib.stream(out),
            ),
            "ctx_scale_bwd",
        )
    return dout, dlse


@_ctx_scale_bwd_op.register_fake
def _(out, lse, ln_pad, dy):
    return torch.empty_like(out), torch.empty_like(lse)


def _ctx_scale_setup(ctx, inputs, output):
    out, lse, ln_pad = inputs
    ctx.save_for_backward(out, lse, ln_pad)


def _ctx_scale_backward(ctx, dy):
    out, lse, ln_pad = ctx.saved_tensors
    dout, dlse = _ctx_scale_bwd_op(out, lse, ln_pad, dy)
    return dout, dlse, None


torch.library.register_autograd(
    "anima_flat::ctx_scale", _ctx_scale_backward, setup_context=_ctx_scale_setup
)


def ctx_scale(out, lse, ln_pad):
    """Rescale trimmed-context attention output to match the zero-padded context.

    Args:
        out: `[B, S, H, hd]` attention output over the kept keys.
        lse: `[B, H, S]` its log-sum-exp.
        ln_pad: `[B]` log of the number of removed padding keys (-inf: none).

    Returns:
        `out * 1/(1 + exp(ln_pad - lse))`, same shape and dtype as `out`.
    """
    _check(out, lse, ln_pad)
    if out.ndim != 4 or lse.shape != (out.shape[0], out.shape[2], out.shape[1]):
        raise ValueError("out must be [B, S, H, hd] and lse [B, H, S]")
    return _ctx_scale(out.contiguous(), lse.float().contiguous(), ln_pad.float().contiguous())
