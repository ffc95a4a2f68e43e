"""Fused input projections of the attention block (inference), opt-in.

Not part of the reference's API and not imported by the package: import
`anima_flat_amd.kernels.proj` to use it. Its op lives in the `anima_flat_amd::`
namespace so it cannot collide with an `anima_flat::` op.

`qkv_proj_norm_rope` = the block's `b.qkv(hid)` projection followed by
`qkv_norm_rope` (src/model.py:308-316) as one kernel (aa_qkv_proj_norm_rope):
the [B, S, 3 * D] projection output stays on chip, q and k are RMS-normalised
and rotated in the GEMM's epilogue, v is written as projected.
"""

from __future__ import annotations

import torch

from .. import _lib
from .common import _check, custom_op
from .rope import _check_hd, _f32


@custom_op("anima_flat_amd::qkv_proj_norm_rope", mutates_args=())
def _qkv_proj_norm_rope(
    hid: torch.Tensor,
    weight: torch.Tensor,
    q_weight: torch.Tensor,
    k_weight: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    heads: int,
    eps: float,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    B, S, D = hid.shape
    hd = 2 * cos.shape[1]
    q = hid.new_empty((B, S, heads, hd))
    k = torch.empty_like(q)
    v = torch.empty_like(q)
    with torch.cuda.device(hid.device):
        _lib.check(
            _lib.lib().aa_qkv_proj_norm_rope(
                hid.data_ptr(),
                hid.stride(1),
                weight.data_ptr(),
                q.data_ptr(),
                k.data_ptr(),
                v.data_ptr(),
                _f32(q_weight).data_ptr(),
                _f32(k_weight).data_ptr(),
                _f32(cos).data_ptr(),
                _f32(sin).data_ptr(),
                B,
                S,
                heads,
                hd,
                eps,
                _lib.dtype_code(hid),
                _lib.stream(hid),
            ),
            "qkv_proj_norm_rope",
        )
    return q, k, v


@_qkv_proj_norm_rope.register_fake
def _(hid, weight, q_weight, k_weight, cos, sin, heads, eps):
    B, S, _ = hid.shape
    q = hid.new_empty((B, S, heads, 2 * cos.shape[1]))
    return q, torch.empty_like(q), torch.empty_like(q)


def qkv_proj_norm_rope(hid, weight, q_weight, k_weight, cos, sin, heads, eps=1e-5):
    """`qkv_norm_rope(F.linear(hid, weight), ...)` as one kernel (the block's
    `b.qkv` projection followed by the prologue, src/model.py:308-316), with the
    projection output kept on chip. Inference only (no autograd).

    Args:
        hid: `[B, S, heads * head_dim]` bf16; rows may be strided (last-dim stride 1).
        weight: `[3 * heads * head_dim, heads * head_dim]` bf16, contiguous (nn.Linear, no bias).
        q_weight, k_weight, cos, sin, heads, eps: as for `qkv_norm_rope`.

    Returns:
        `(q, k, v)`, each a contiguous `[B, S, heads, head_dim]`.
    """
    _check(hid, weight, q_weight, k_weight, cos, sin)
    hd = 2 * cos.shape[1]
    D = heads * hd
    if hid.ndim != 3 or hid.shape[-1] != D or hid.stride(-1) != 1 or hid.stride(0) != hid.shape[1] * hid.stride(1):
        raise ValueError("hid must be [B, S, heads * head_dim] with unit last-dim stride and uniform rows")
    if not weight.is_contiguous() or tuple(weight.shape) != (3 * D, D) or weight.dtype != hid.dtype:
        raise ValueError("weight must be a contiguous [3 * heads * head_dim, heads * head_dim] matrix of hid's dtype")
    if cos.shape != sin.shape or cos.shape[0] != hid.shape[1] or (cos.shape[1] & (cos.shape[1] - 1)):
        raise ValueError("cos/sin must be [S, head_dim // 2] with a power-of-two width")
    _check_hd(hd)
    if torch.is_grad_enabled() and (hid.requires_grad or weight.requires_grad or q_weight.requires_grad):
        raise RuntimeError("qkv_proj_norm_rope has no backward: use F.linear + qkv_norm_rope for training")
    return _qkv_proj_norm_rope(
        hid, weight, q_weight.contiguous(), k_weight.contiguous(), cos.contiguous(), sin.contiguous(), heads, eps
    )
