"""Fused input projections of the attention block (inference), opt-in.

Not part of the reference's API and not imported by the package: import
`anima_flat_amd.kernels.proj` to use it. Its ops live in the `anima_flat_amd::`
namespace so they cannot collide with an `anima_flat::` op.

One GEMM kernel (csrc/qkv_proj.hip) with the normalisation in its epilogue, so
the projection output never reaches memory:
  qkv_proj_norm_rope  the block's `b.qkv(hid)` + `qkv_norm_rope` (src/model.py:308-316)
  proj_head_norm      `b.xq(hid)` + `head_norm` (src/model.py:324)
  kv_proj_norm        `b.xkv(ctx)` + the key-side RMSNorm (src/model.py:256-258)
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
    qw, kw, c32, s32 = _f32(q_weight), _f32(k_weight), _f32(cos), _f32(sin)
    with torch.cuda.device(hid.device):
        for sl, rows, rs in _row_launches(hid):
            _lib.check(
                _lib.lib().aa_qkv_proj_norm_rope(
                    rows.data_ptr(), rs, weight.data_ptr(), q[sl].data_ptr(), k[sl].data_ptr(),
                    v[sl].data_ptr(), qw.data_ptr(), kw.data_ptr(), c32.data_ptr(), s32.data_ptr(),
                    rows.shape[0], S, heads, hd, eps, _lib.dtype_code(hid), _lib.stream(hid),
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
        hid: `[B, S, heads * head_dim]` bf16, last-dim stride 1; rows and batch items may
            be strided.
        weight: `[3 * heads * head_dim, heads * head_dim]` bf16, contiguous (nn.Linear, no bias).
        q_weight, k_weight, cos, sin, heads, eps: as for `qkv_norm_rope`.

    Returns:
        `(q, k, v)`, each a contiguous `[B, S, heads, head_dim]`.
    """
    _check(hid, weight, q_weight, k_weight, cos, sin)
    hd = 2 * cos.shape[1]
    D = heads * hd
    if not _rows_ok(hid) or hid.shape[-1] != D:
        raise ValueError("hid must be [B, S, heads * head_dim] with unit last-dim stride")
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


def _rows_ok(x: torch.Tensor) -> bool:
    """[B, S, K] with unit last-dim stride (any batch and row strides)."""
    return x.ndim == 3 and x.stride(-1) == 1


def _row_launches(x: torch.Tensor):
    """How to hand the rows of a [B, S, K] input to the C ABI, which addresses
    them as B * S rows at one row stride: a list of (batch slice, rows view,
    row stride). One launch when the rows are uniform (always so for B == 1:
    the batch stride then addresses nothing); otherwise one per batch item,
    each item's S rows being uniform. A sequence-trimmed view such as
    `ctx[:, :keep]` (src/model.py:251) has stride(0) = S_full * K, not keep * K.
    """
    B, S, K = x.shape
    if S == 1:
        if B == 1 or x.stride(0) >= K:
            return [(slice(None), x, x.stride(0) if B > 1 else K)]
        return [(slice(b, b + 1), x[b : b + 1], K) for b in range(B)]
    if B == 1 or x.stride(0) == S * x.stride(1):
        return [(slice(None), x, x.stride(1))]
    return [(slice(b, b + 1), x[b : b + 1], x.stride(1)) for b in range(B)]


@custom_op("anima_flat_amd::proj_head_norm", mutates_args=())
def _proj_head_norm(
    x: torch.Tensor, weight: torch.Tensor, norm_weight: torch.Tensor, heads: int, eps: float
) -> torch.Tensor:
    B, S, K = x.shape
    hd = norm_weight.numel()
    y = x.new_empty((B, S, heads, hd))
    nw = _f32(norm_weight)
    with torch.cuda.device(x.device):
        for sl, rows, rs in _row_launches(x):
            _lib.check(
                _lib.lib().aa_proj_head_norm(
                    rows.data_ptr(), rs, weight.data_ptr(), K, y[sl].data_ptr(), nw.data_ptr(),
                    rows.shape[0], S, heads, hd, eps, _lib.dtype_code(x), _lib.stream(x),
                ),
                "proj_head_norm",
            )
    return y


@_proj_head_norm.register_fake
def _(x, weight, norm_weight, heads, eps):
    B, S, _ = x.shape
    return x.new_empty((B, S, heads, norm_weight.numel()))


def proj_head_norm(x, weight, norm_weight, heads, eps=1e-5):
    """`head_norm(F.linear(x, weight), norm_weight, heads, eps)` as one kernel: the
    cross-attention query projection and its per-head RMSNorm
    (`head_norm(b.xq(hid), b.xq_norm, c.heads, c.qk_eps)`, src/model.py:324), with
    the projection output kept on chip. Inference only (no autograd).

    Args:
        x: `[B, S, K]` bf16 (K a multiple of 32), last-dim stride 1; rows and batch items
            may be strided.
        weight: `[heads * head_dim, K]` bf16, contiguous (nn.Linear, no bias).
        norm_weight: RMSNorm weight `[head_dim]`.
        heads, eps: as for `head_norm`.

    Returns:
        `[B, S, heads, head_dim]`, contiguous.
    """
    _check(x, weight, norm_weight)
    hd = norm_weight.numel()
    _check_hd(hd)
    if not _rows_ok(x):
        raise ValueError("x must be [B, S, K] with unit last-dim stride")
    if not weight.is_contiguous() or tuple(weight.shape) != (heads * hd, x.shape[-1]) or weight.dtype != x.dtype:
        raise ValueError("weight must be a contiguous [heads * head_dim, K] matrix of x's dtype")
    if torch.is_grad_enabled() and (x.requires_grad or weight.requires_grad or norm_weight.requires_grad):
        raise RuntimeError("proj_head_norm has no backward: use F.linear + head_norm for training")
    return _proj_head_norm(x, weight, norm_weight.contiguous(), heads, eps)


@custom_op("anima_flat_amd::kv_proj_norm", mutates_args=())
def _kv_proj_norm(
    ctx: torch.Tensor, weight: torch.Tensor, k_weight: torch.Tensor, heads: int, eps: float
) -> tuple[torch.Tensor, torch.Tensor]:
    B, S, K = ctx.shape
    hd = k_weight.numel()
    k = ctx.new_empty((B, S, heads, hd))
    v = torch.empty_like(k)
    kw = _f32(k_weight)
    with torch.cuda.device(ctx.device):
        for sl, rows, rs in _row_launches(ctx):
            _lib.check(
                _lib.lib().aa_kv_proj_norm(
                    rows.data_ptr(), rs, weight.data_ptr(), K, k[sl].data_ptr(), v[sl].data_ptr(),
                    kw.data_ptr(), rows.shape[0], S, heads, hd, eps, _lib.dtype_code(ctx),
                    _lib.stream(ctx),
                ),
                "kv_proj_norm",
            )
    return k, v


@_kv_proj_norm.register_fake
def _(ctx, weight, k_weight, heads, eps):
    B, S, _ = ctx.shape
    k = ctx.new_empty((B, S, heads, k_weight.numel()))
    return k, torch.empty_like(k)


def kv_proj_norm(ctx, weight, k_weight, heads, eps=1e-5):
    """One layer's context keys and values with the key-side RMSNorm fused
    (src/model.py:256-258, in encode_context):
    `k, v = b.xkv(ctx).view(B, S, 2, heads, hd).unbind(2)` then
    `k = F.rms_norm(k, (hd,), b.xk_norm.to(k.dtype), eps)`, as one kernel with the
    projection output kept on chip. Inference only (no autograd).

    Args:
        ctx: `[B, S, K]` bf16 text context (K = text_dim, a multiple of 32), last-dim
            stride 1; rows and batch items may be strided, e.g. the sequence-trimmed
            `ctx[:, :keep]` of `trim_context` (src/model.py:248-253).
        weight: `[2 * heads * head_dim, K]` bf16, contiguous (nn.Linear, no bias).
        k_weight: RMSNorm weight `[head_dim]`; applied in the activation dtype as
            F.rms_norm does, so pass `b.xk_norm.to(ctx.dtype)` as the reference does.
        heads, eps: as for `head_norm`.

    Returns:
        `(k, v)`, each a contiguous `[B, S, heads, head_dim]`.
    """
    _check(ctx, weight, k_weight)
    hd = k_weight.numel()
    _check_hd(hd)
    if not _rows_ok(ctx):
        raise ValueError("ctx must be [B, S, K] with unit last-dim stride")
    if not weight.is_contiguous() or tuple(weight.shape) != (2 * heads * hd, ctx.shape[-1]) or weight.dtype != ctx.dtype:
        raise ValueError("weight must be a contiguous [2 * heads * head_dim, K] matrix of ctx's dtype")
    if torch.is_grad_enabled() and (ctx.requires_grad or weight.requires_grad or k_weight.requires_grad):
        raise RuntimeError("kv_proj_norm has no backward: use F.linear + F.rms_norm for training")
    return _kv_proj_norm(ctx, weight, k_weight.contiguous(), heads, eps)
