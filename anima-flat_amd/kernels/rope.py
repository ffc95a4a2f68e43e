"""QK-RMSNorm + 3D RoPE prologue and per-head RMSNorm on MI355X.

Drop-in for anima-flat's src/kernels/rope.py: same public functions
(`qkv_norm_rope`, `head_norm`, rope.py:616-652), the same torch.library ops
(`anima_flat::qkv_norm_rope`, `qkv_norm_rope_v`, `qkv_norm_rope_bwd`,
`head_norm`, `head_norm_bwd`) with their schemas, fakes and autograd
registrations, and the same validation errors. The Triton kernels are replaced
by HIP kernels of libanima_attn.so (aa_qkv_norm_rope_fwd/_bwd,
aa_head_norm_fwd/_bwd).

Per (token, head): rstd = rsqrt(mean(x^2) + eps) in fp32; y = x * rstd * w
rounded to the activation dtype; then rotate-half RoPE on pairs
(y[i], y[i + hd/2]) with cos/sin[position, i], position = token index within
its sequence. V needs no norm or rotation.
"""

from __future__ import annotations

import torch

from .. import _lib
from .common import _check, custom_op


def _f32(t: torch.Tensor) -> torch.Tensor:
    return t.to(torch.float32).contiguous()


def _check_hd(hd: int) -> None:
    if hd != 128:
        raise ValueError(f"head_dim {hd} is not supported (128 only)")


# ----------------------------------------------------------------- forward --


def _launch_qkv(qkv, q_weight, k_weight, cos, sin, heads, eps, with_v):
    B, S, _ = qkv.shape
    half = cos.shape[1]
    hd = 2 * half
    _check_hd(hd)
    q = qkv.new_empty((B, S, heads, hd))
    k = torch.empty_like(q)
    v = torch.empty_like(q) if with_v else None
    with torch.cuda.device(qkv.device):
        _lib.check(
            _lib.lib().aa_qkv_norm_rope_fwd(
                qkv.data_ptr(),
                q.data_ptr(),
                k.data_ptr(),
                _lib.ptr(v),
                _f32(q_weight).data_ptr(),
                _f32(k_weight).data_ptr(),
                _f32(cos).data_ptr(),
                _f32(sin).data_ptr(),
                B,
                S,
                heads,
                hd,
                eps,
                _lib.dtype_code(qkv),
                _lib.stream(qkv),
            ),
            "qkv_norm_rope",
        )
    return q, k, v


@custom_op("anima_flat::qkv_norm_rope", mutates_args=())
def _qkv_norm_rope(
    qkv: torch.Tensor,
    q_weight: torch.Tensor,
    k_weight: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    heads: int,
    eps: float,
) -> tuple[torch.Tensor, torch.Tensor]:
    q, k, _ = _launch_qkv(qkv, q_weight, k_weight, cos, sin, heads, eps, with_v=False)
    return q, k


@_qkv_norm_rope.register_fake
def _(qkv, q_weight, k_weight, cos, sin, heads, eps):
    B, S, _ = qkv.shape
    q = qkv.new_empty((B, S, heads, 2 * cos.shape[1]))
    return q, torch.empty_like(q)


@custom_op("anima_flat::head_norm", mutates_args=())
def _head_norm(x: torch.Tensor, weight: torch.Tensor, heads: int, eps: float) -> torch.Tensor:
    B, S, _ = x.shape
    hd = weight.numel()
    _check_hd(hd)
    y = x.new_empty((B, S, heads, hd))
    with torch.cuda.device(x.device):
        _lib.check(
            _lib.lib().aa_head_norm_fwd(
                x.data_ptr(),
                y.data_ptr(),
                _f32(weight).data_ptr(),
                B,
                S,
                heads,
                hd,
                eps,
                _lib.dtype_code(x),
                _lib.stream(x),
            ),
            "head_norm",
        )
    return y


@_head_norm.register_fake
def _(x, weight, heads, eps):
    return x.new_empty((x.shape[0], x.shape[1], heads, weight.numel()))


# ---------------------------------------------------------------- backward --


def _head_norm_bwd(x, dy, weight, heads, eps):
    B, S, _ = x.shape
    hd = weight.numel()
    _check_hd(hd)
    dy = dy.contiguous()
    dx = torch.empty_like(x)
    dw = torch.empty(hd, dtype=torch.float32, device=x.device)
    ws_bytes = _lib.lib().aa_head_norm_bwd_workspace(B, S, heads, hd)
    ws = torch.empty(max(ws_bytes // 4, 1), dtype=torch.float32, device=x.device)
    with torch.cuda.device(x.device):
        _lib.check(
            _lib.lib().aa_head_norm_bwd(
                x.data_ptr(),
                dy.data_ptr(),
                dx.data_ptr(),
                _f32(weight).data_ptr(),
                dw.data_ptr(),
                ws.data_ptr(),
                ws_bytes,
                B,
                S,
                heads,
                hd,
                eps,
                _lib.dtype_code(x),
                _lib.stream(x),
            ),
            "head_norm_bwd",
        )
    return dx, dw.to(weight.dtype)


@custom_op("anima_flat::head_norm_bwd", mutates_args=())
def _head_norm_bwd_op(
    x: torch.Tensor, dy: torch.Tensor, weight: torch.Tensor, heads: int, eps: float
) -> tuple[torch.Tensor, torch.Tensor]:
    return _head_norm_bwd(x, dy, weight, heads, eps)


@_head_norm_bwd_op.register_fake
def _(x, dy, weight, heads, eps):
    return torch.empty_like(x), torch.empty_like(weight)


def _head_norm_setup(ctx, inputs, output):
    x, weight, heads, eps = inputs
    ctx.save_for_backward(x, weight)
    ctx.heads = heads
    ctx.eps = eps


def _head_norm_backward(ctx, dy):
    x, weight = ctx.saved_tensors
    dx, dw = _head_norm_bwd_op(x, dy, weight, ctx.heads, ctx.eps)
    return dx, dw, None, None


torch.library.register_autograd(
    "anima_flat::head_norm", _head_norm_backward, setup_context=_head_norm_setup
)


@custom_op("anima_flat::qkv_norm_rope_v", mutates_args=())
def _qkv_norm_rope_v(
    qkv: torch.Tensor,
    q_weight: torch.Tensor,
    k_weight: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    heads: int,
    eps: float,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    q, k, v = _launch_qkv(qkv, q_weight, k_weight, cos, sin, heads, eps, with_v=True)
    return q, k, v


@_qkv_norm_rope_v.register_fake
def _(qkv, q_weight, k_weight, cos, sin, heads, eps):
    B, S, _ = qkv.shape
    q = qkv.new_empty((B, S, heads, 2 * cos.shape[1]))
    return q, torch.empty_like(q), torch.empty_like(q)


def _qkv_norm_rope_setup(ctx, inputs, output):
    qkv, q_weight, k_weight, cos, sin, heads, eps = inputs
    ctx.save_for_backward(qkv, q_weight, k_weight, cos, sin)
    ctx.heads = heads
    ctx.eps = eps


def _qkv_norm_rope_bwd(qkv, dq, dk, dv, q_weight, k_weight, cos, sin, heads, eps):
    B, S, _ = qkv.shape
    half = cos.shape[1]
    hd = 2 * half
    _check_hd(hd)
    dq, dk, dv = dq.contiguous(), dk.contiguous(), dv.contiguous()
    dqkv = torch.empty_like(qkv)
    dqw = torch.empty(hd, dtype=torch.float32, device=qkv.device)
    dkw = torch.empty(hd, dtype=torch.float32, device=qkv.device)
    ws_bytes = _lib.lib().aa_qkv_norm_rope_bwd_workspace(B, S, heads, hd)
    ws = torch.empty(max(ws_bytes // 4, 1), dtype=torch.float32, device=qkv.device)
    with torch.cuda.device(qkv.device):
        _lib.check(
            _lib.lib().aa_qkv_norm_rope_bwd(
                qkv.data_ptr(),
                dq.data_ptr(),
                dk.data_ptr(),
                dv.data_ptr(),
                dqkv.data_ptr(),
                _f32(q_weight).data_ptr(),
                _f32(k_weight).data_ptr(),
                _f32(cos).data_ptr(),
                _f32(sin).data_ptr(),
                dqw.data_ptr(),
                dkw.data_ptr(),
                ws.data_ptr(),
                ws_bytes,
                B,
                S,
                heads,
                hd,
                eps,
                _lib.dtype_code(qkv),
                _lib.stream(qkv),
            ),
            "qkv_norm_rope_bwd",
        )
    return dqkv, dqw.to(q_weight.dtype), dkw.to(k_weight.dtype)


@custom_op("anima_flat::qkv_norm_rope_bwd", mutates_args=())
def _qkv_norm_rope_bwd_op(
    qkv: torch.Tensor,
    dq: torch.Tensor,
    dk: torch.Tensor,
    dv: torch.Tensor,
    q_weight: torch.Tensor,
    k_weight: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    heads: int,
    eps: float,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    return _qkv_norm_rope_bwd(qkv, dq, dk, dv, q_weight, k_weight, cos, sin, heads, eps)


@_qkv_norm_rope_bwd_op.register_fake
def _(qkv, dq, dk, dv, q_weight, k_weight, cos, sin, heads, eps):
    return torch.empty_like(qkv), torch.empty_like(q_weight), torch.empty_like(k_weight)


def _qkv_norm_rope_backward(ctx, dq, dk, dv):
    qkv, q_weight, k_weight, cos, sin = ctx.saved_tensors
    dqkv, dqw, dkw = _qkv_norm_rope_bwd_op(
        qkv, dq, dk, dv, q_weight, k_weight, cos, sin, ctx.heads, ctx.eps
    )
    return dqkv, dqw, dkw, None, None, None, None


torch.library.register_autograd(
    "anima_flat::qkv_norm_rope_v",
    _qkv_norm_rope_backward,
    setup_context=_qkv_norm_rope_setup,
)


# ------------------------------------------------------------- public API --


def qkv_norm_rope(qkv, q_weight, k_weight, cos, sin, heads, eps=1e-5):
    """Split a fused QKV projection into heads, RMS-normalise q and k, rotate them.

    Mirrors src/kernels/rope.py:616-645: with autograd needed (qkv or q_weight
    requiring grad) V is copied by the kernel (op qkv_norm_rope_v); otherwise
    V is returned as a strided view of `qkv` and only q, k are written.

    Args:
        qkv: `[B, S, 3 * heads * head_dim]`, contiguous.
        q_weight, k_weight: RMSNorm weights `[head_dim]`.
        cos, sin: Rotary tables `[S, head_dim // 2]` (power-of-two width).
        heads: Number of heads.
        eps: RMSNorm epsilon.

    Returns:
        `(q, k, v)`, each `[B, S, heads, head_dim]`.
    """
    _check(qkv, q_weight, k_weight, cos, sin)
    if (
        not qkv.is_contiguous()
        or qkv.ndim != 3
        or qkv.shape[-1] != 3 * heads * 2 * cos.shape[1]
    ):
        raise ValueError("qkv must be contiguous [B, S, 3 * heads * head_dim]")
    if (
        cos.shape != sin.shape
        or cos.shape[0] != qkv.shape[1]
        or (cos.shape[1] & (cos.shape[1] - 1))
    ):
        raise ValueError("cos/sin must be [S, head_dim // 2] with a power-of-two width")
    args = (
        qkv,
        q_weight.contiguous(),
        k_weight.contiguous(),
        cos.contiguous(),
        sin.contiguous(),
        heads,
        eps,
    )
    if torch.is_grad_enabled() and (qkv.requires_grad or q_weight.requires_grad):
        return _qkv_norm_rope_v(*args)
    q, k = _qkv_norm_rope(*args)
    # V needs no norm or rotation: a strided view of qkv, read in place by attention.
    B, S, _ = qkv.shape
    v = qkv.view(B, S, 3, heads, 2 * cos.shape[1])[:, :, 2]
    return q, k, v


def head_norm(x, weight, heads, eps=1e-5):
    """Per-head RMSNorm of `x` `[B, S, heads * head_dim]` -> `[B, S, heads, head_dim]`
    (src/kernels/rope.py:648-652)."""
    _check(x, weight)
    if not x.is_contiguous() or x.shape[-1] != heads * weight.numel():
        raise ValueError("x must be contiguous [B, S, heads * head_dim]")
    return _head_norm(x, weight.contiguous(), heads, eps)
