"""Non-causal multi-head attention on MI355X, drop-in for anima-flat's src/attention.py.

Same public functions (`use_fa4`, `attention`, `cross_attention_trimmed`) and
the same torch.library ops (`anima_flat::fa_fwd`, `fa_fwd_nolse`, `fa_fwd_k`,
`fa_bwd`) with the same schemas, fake registrations and autograd wiring as
src/attention.py:21-180. The FlashAttention-4 calls are replaced by the HIP
kernels of libanima_attn.so (aa_attn_fwd / aa_attn_bwd).

One code path: where the reference falls back to torch SDPA
(src/attention.py:150-153) these functions raise instead. The environment
variable ANIMA_FLAT_ATTENTION=sdpa still makes `use_fa4` return False, which
the model uses to decide whether to trim the text context.
"""

from __future__ import annotations

import functools
import math
import os

import torch

from . import _lib
from .kernels.common import _check, custom_op


@functools.cache
def _capable(index: int) -> bool:
    """True for a gfx950 (MI350-series) device: the kernels are built for it only."""
    props = torch.cuda.get_device_properties(index)
    return getattr(props, "gcnArchName", "").split(":")[0] == "gfx950"


def use_fa4(t: torch.Tensor) -> bool:
    """Decide whether the fused attention kernels can serve tensors like `t`.

    Mirrors src/attention.py:21-40. The `ANIMA_FLAT_ATTENTION=sdpa` environment
    variable makes this return False (the model then skips context trimming).

    Args:
        t: Representative attention input; its device and dtype are checked.

    Returns:
        True if libanima_attn.so loads, `t` is a bf16 tensor on a GPU, and the
        GPU is gfx950; False otherwise.
    """
    if os.environ.get("ANIMA_FLAT_ATTENTION", "fa4") == "sdpa":
        return False
    return (
        _lib.available()
        and t.is_cuda
        and t.dtype == torch.bfloat16
        and _capable(t.device.index if t.device.index is not None else torch.cuda.current_device())
    )


# ------------------------------------------------------------------ launch --


def _kernel_ready(t: torch.Tensor) -> bool:
    s = t.stride()
    return (
        s[3] == 1
        and t.data_ptr() % 16 == 0
        and s[0] % 8 == 0
        and s[1] % 8 == 0
        and s[2] % 8 == 0
    )


def _prep(t: torch.Tensor) -> torch.Tensor:
    """A view the kernels accept: last-dim stride 1, 16-byte aligned pointer, other
    strides multiples of 8 elements. Copies only when `t` is not already one."""
    if t.numel() == 0 or _kernel_ready(t):
        return t
    t = t.contiguous()
    if not _kernel_ready(t):
        t = t.clone(memory_format=torch.contiguous_format)
    return t


def _validate(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, head_dims=(128,)) -> None:
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("q, k, v must be [B, S, H, hd]")
    if k.shape != v.shape:
        raise ValueError(f"k {tuple(k.shape)} and v {tuple(v.shape)} must have the same shape")
    if q.shape[0] != k.shape[0] or q.shape[2] != k.shape[2] or q.shape[3] != k.shape[3]:
        raise ValueError(
            f"q {tuple(q.shape)} and k {tuple(k.shape)} disagree on batch, heads or head_dim"
        )
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError("q, k, v must share a dtype")
    if not (q.device == k.device == v.device):
        raise ValueError("q, k, v must be on one device")
    _lib.dtype_code(q)
    if q.shape[3] not in head_dims:
        raise ValueError(f"head_dim {q.shape[3]} is not supported ({' or '.join(map(str, head_dims))} only)")


def _fwd_args(q, k, v, out, lse, seqused_k, ln_pad) -> _lib.AttnFwdArgs:
    B, Sq, H, hd = q.shape
    a = _lib.AttnFwdArgs()
    a.q, a.k, a.v, a.out = q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr()
    a.lse = _lib.ptr(lse)
    a.seqused_k = _lib.ptr(seqused_k)
    a.ln_pad = _lib.ptr(ln_pad)
    a.q_stride = _lib.c_strides(_lib.bshd_strides(q))
    a.k_stride = _lib.c_strides(_lib.bshd_strides(k))
    a.v_stride = _lib.c_strides(_lib.bshd_strides(v))
    a.out_stride = _lib.c_strides(_lib.bshd_strides(out))
    a.B, a.Sq, a.Sk, a.H, a.hd = B, Sq, k.shape[1], H, hd
    a.softmax_scale = 1.0 / math.sqrt(hd)
    a.dtype = _lib.dtype_code(q)
    return a


@_lib.on_device
def _launch_fwd(q, k, v, *, want_lse, seqused_k=None, ln_pad=None, head_dims=(128,)):
    """Runs aa_attn_fwd; returns (out [B,Sq,H,hd] contiguous, lse [B,H,Sq] or None)."""
    _validate(q, k, v, head_dims)
    q, k, v = _prep(q), _prep(k), _prep(v)
    B, Sq, H, _ = q.shape
    out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    lse = torch.empty((B, H, Sq), dtype=torch.float32, device=q.device) if want_lse else None
    if seqused_k is not None:
        if seqused_k.shape != (B,):
            raise ValueError(f"seqused_k must be [B]={B}, got {tuple(seqused_k.shape)}")
        seqused_k = seqused_k.to(device=q.device, dtype=torch.int32).contiguous()
    if ln_pad is not None:
        if ln_pad.shape != (B,):
            raise ValueError(f"ln_pad must be [B]={B}, got {tuple(ln_pad.shape)}")
        ln_pad = ln_pad.to(device=q.device, dtype=torch.float32).contiguous()
    args = _fwd_args(q, k, v, out, lse, seqused_k, ln_pad)
    ws_bytes = _lib.lib().aa_attn_fwd_workspace(B, Sq, k.shape[1], H, q.shape[3])
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=q.device) if ws_bytes else None
    if ws is not None:
        args.workspace, args.workspace_bytes = ws.data_ptr(), ws_bytes
    _lib.call_attn_fwd(args, _lib.stream(q))
    return out, lse


@_lib.on_device
def _launch_bwd(dout, q, k, v, out, lse):
    _validate(q, k, v)
    if dout.shape != q.shape or out.shape != q.shape:
        raise ValueError("dout and out must have q's shape")
    B, Sq, H, hd = q.shape
    if lse.shape != (B, H, Sq):
        raise ValueError(f"lse must be [B, H, Sq]={(B, H, Sq)}, got {tuple(lse.shape)}")
    dout = _prep(dout.contiguous())
    q, k, v, out = _prep(q), _prep(k), _prep(v), _prep(out)
    lse = lse.to(torch.float32).contiguous()
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    dq, dk, dv = _prep(dq), _prep(dk), _prep(dv)
    a = _lib.AttnBwdArgs()
    a.dout, a.q, a.k, a.v, a.out = (t.data_ptr() for t in (dout, q, k, v, out))
    a.lse = lse.data_ptr()
    a.dq, a.dk, a.dv = dq.data_ptr(), dk.data_ptr(), dv.data_ptr()
    for name, t in (
        ("dout_stride", dout),
        ("q_stride", q),
        ("k_stride", k),
        ("v_stride", v),
        ("out_stride", out),
        ("dq_stride", dq),
        ("dk_stride", dk),
        ("dv_stride", dv),
    ):
        setattr(a, name, _lib.c_strides(_lib.bshd_strides(t)))
    a.B, a.Sq, a.Sk, a.H, a.hd = B, Sq, k.shape[1], H, hd
    a.softmax_scale = 1.0 / math.sqrt(hd)
    a.dtype = _lib.dtype_code(q)
    ws_bytes = _lib.lib().aa_attn_bwd_workspace(B, Sq, k.shape[1], H, hd)
    ws = torch.empty(max(ws_bytes // 4, 1), dtype=torch.float32, device=q.device)
    _lib.call_attn_bwd(a, ws, ws_bytes, _lib.stream(q))
    return dq, dk, dv


# --------------------------------------------------------------------- ops --


@custom_op("anima_flat::fa_fwd", mutates_args=())
def _fa_fwd(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor
) -> tuple[torch.Tensor, torch.Tensor]:
    out, lse = _launch_fwd(q, k, v, want_lse=True)
    return out, lse


@_fa_fwd.register_fake
def _(q, k, v):
    return torch.empty_like(q), q.new_empty(
        (q.shape[0], q.shape[2], q.shape[1]), dtype=torch.float32
    )


@custom_op("anima_flat::fa_fwd_nolse", mutates_args=())
def _fa_fwd_nolse(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    out, _ = _launch_fwd(q, k, v, want_lse=False)
    return out


@_fa_fwd_nolse.register_fake
def _(q, k, v):
    return q.new_empty(q.shape)


@custom_op("anima_flat::fa_fwd_k", mutates_args=())
def _fa_fwd_k(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, seqused_k: torch.Tensor
) -> tuple[torch.Tensor, torch.Tensor]:
    out, lse = _launch_fwd(q, k, v, want_lse=True, seqused_k=seqused_k)
    return out, lse


@_fa_fwd_k.register_fake
def _(q, k, v, seqused_k):
    return torch.empty_like(q), q.new_empty(
        (q.shape[0], q.shape[2], q.shape[1]), dtype=torch.float32
    )


@custom_op("anima_flat_amd::fa_fwd_k_ctx", mutates_args=())
def _fa_fwd_k_ctx(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    seqused_k: torch.Tensor,
    ln_pad: torch.Tensor,
) -> torch.Tensor:
    """Key-length-masked attention with the padding correction applied in the
    kernel epilogue: fa_fwd_k followed by ctx_scale in one launch."""
    out, _ = _launch_fwd(q, k, v, want_lse=False, seqused_k=seqused_k, ln_pad=ln_pad)
    return out


@_fa_fwd_k_ctx.register_fake
def _(q, k, v, seqused_k, ln_pad):
    return q.new_empty(q.shape)


@custom_op("anima_flat::fa_bwd", mutates_args=())
def _fa_bwd(
    dout: torch.Tensor,
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    out: torch.Tensor,
    lse: torch.Tensor,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    return _launch_bwd(dout, q, k, v, out, lse)


@_fa_bwd.register_fake
def _(dout, q, k, v, out, lse):
    return torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)


def _setup_context(ctx, inputs, output):
    q, k, v = inputs
    out, lse = output
    ctx.mark_non_differentiable(lse)
    # The backward never reads the LSE's gradient: without this autograd fills
    # a zero tensor for it (one extra kernel launch per backward).
    ctx.set_materialize_grads(False)
    ctx.save_for_backward(q, k, v, out, lse)


def _backward(ctx, dout, dlse):
    q, k, v, out, lse = ctx.saved_tensors
    if dout is None:  # only possible without materialized grads: no gradient reaches out
        return None, None, None
    return _fa_bwd(dout, q, k, v, out, lse)


_fa_fwd.register_autograd(_backward, setup_context=_setup_context)


# ------------------------------------------------------------- public API --


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """Full (non-causal) multi-head attention (src/attention.py:126-153).

    Differentiable. Inputs are not copied when they are strided views with
    last-dim stride 1, 16-byte-aligned pointers and other strides that are
    multiples of 8 elements (else they are copied first). The softmax LSE is
    only computed when autograd needs it.

    Args:
        q: Queries, shape `[B, Sq, H, hd]`.
        k: Keys, shape `[B, Sk, H, hd]`.
        v: Values, shape `[B, Sk, H, hd]`.

    Returns:
        Attention output with heads merged, shape `[B, Sq, H * hd]`, dtype of `q`.

    Raises:
        ValueError: for CPU tensors, a dtype other than bf16, head_dim other
            than 128, or inconsistent shapes.
        RuntimeError: if libanima_attn.so is missing or a launch fails.
    """
    _check(q, k, v)
    if torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad):
        out, _ = _fa_fwd(q, k, v)
    else:
        out = _fa_fwd_nolse(q, k, v)
    return out.flatten(2)


def cross_attention_trimmed(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    seqused_k: torch.Tensor,
    ln_pad: torch.Tensor,
) -> torch.Tensor:
    """Cross-attention over a trimmed key/value context, corrected for the removed
    padding (src/attention.py:156-180).

    Only the first `seqused_k[b]` keys of batch item `b` are attended; the output
    is rescaled by 1/(1 + exp(ln_pad - lse)) so it matches attention over the
    full zero-padded context. Mask and correction run in one kernel.

    Args:
        q: Queries, shape `[B, Sq, H, hd]`.
        k: Trimmed keys, shape `[B, Sk_trim, H, hd]`.
        v: Trimmed values, shape `[B, Sk_trim, H, hd]`.
        seqused_k: Valid key count per batch item, int32, shape `[B]`.
        ln_pad: `log(S_full - seqused_k)` per batch item, float32, shape `[B]`.

    Returns:
        Attention output with heads merged, shape `[B, Sq, H * hd]`.
    """
    _check(q, k, v, seqused_k, ln_pad)
    return _fa_fwd_k_ctx(q.contiguous(), k, v, seqused_k, ln_pad).flatten(2)
