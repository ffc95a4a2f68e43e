"""Rotary tables and cross-attention context plumbing around the attention path.

Mirrors the parts of anima-flat's src/model.py that feed the path:
  rope_tables      <- model.py:51-84 (3D t/h/w rotary tables for an h x w grid)
  Context          <- model.py:87-119 (per-layer K/V + trim state, `attend`)
  trim_context     <- model.py:247-254 (drop trailing zero padding of the text
                      context; key lengths and log of the removed padding)
  context_lengths  <- model.py:248-253 on the device (aa_context_lengths): the
                      same key lengths and log padding with no host read and no
                      trim (the masked attention reads only the first
                      seqused[b] keys of the untrimmed K/V)

The table formula must reproduce the reference's values exactly, so it
follows the same sequence of float32 operations.
"""

from __future__ import annotations

import torch

from . import _lib
from .attention import attention, cross_attention_trimmed
from .kernels.common import _check


def rope_tables(
    h: int,
    w: int,
    head_dim: int,
    device: str | torch.device,
    rope_scale: tuple = (1.0, 1.0),
) -> tuple[torch.Tensor, torch.Tensor]:
    """3D (time, height, width) rotary tables for an `h x w` token grid (T = 1).

    head_dim splits into a time part (angle 0 for single images) and equal
    height and width parts of dh = head_dim // 6 * 2 dims (21 + 21 slots of the
    64 at head_dim 128, after 22 time slots). Height/width frequencies are
    1 / (10000 * scale^(dh/(dh-2)))^(2i/dh).

    Returns:
        `(cos, sin)`, each float32 `[h * w, head_dim // 2]`, row = y * w + x.
    """
    dh = head_dim // 6 * 2
    dt = head_dim - 2 * dh
    ntk = dh / (dh - 2)
    exponent = torch.arange(0, dh, 2, device=device, dtype=torch.float32) / dh
    inv_h = 1.0 / ((10000.0 * rope_scale[0] ** ntk) ** exponent)
    inv_w = 1.0 / ((10000.0 * rope_scale[1] ** ntk) ** exponent)
    rows = torch.arange(h, device=device, dtype=torch.float32)
    cols = torch.arange(w, device=device, dtype=torch.float32)
    ang_h = torch.outer(rows, inv_h)[:, None, :].expand(h, w, -1)
    ang_w = torch.outer(cols, inv_w)[None, :, :].expand(h, w, -1)
    ang_t = torch.zeros(h, w, dt // 2, device=device)
    angles = torch.cat([ang_t, ang_h, ang_w], dim=-1).reshape(h * w, -1)
    return angles.cos(), angles.sin()


class Context:
    """Per-layer cross-attention keys/values of one text context.

    Attributes:
        kv: Per-layer `(k, v)` pairs, each `[B, S, H, hd]`.
        seqused: Valid context length per batch item (int32 `[B]`) if trimmed, else None.
        ln_pad: log of the number of trimmed padding keys per batch item (`[B]`) if
            trimmed, else None.
    """

    def __init__(
        self,
        kv: list[tuple[torch.Tensor, torch.Tensor]],
        seqused: torch.Tensor | None = None,
        ln_pad: torch.Tensor | None = None,
    ) -> None:
        self.kv = kv
        self.seqused = seqused
        self.ln_pad = ln_pad

    def attend(self, layer: int, q: torch.Tensor) -> torch.Tensor:
        """Cross-attend `q` `[B, Sq, H, hd]` to layer `layer`'s context -> `[B, Sq, H*hd]`."""
        k, v = self.kv[layer]
        if self.seqused is None:
            return attention(q, k, v)
        return cross_attention_trimmed(q, k, v, self.seqused, self.ln_pad)  # type: ignore[arg-type]


def trim_context(ctx: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Drop trailing all-zero rows of a zero-padded text context.

    The length of item b is the 1-based index of its last non-zero row (at
    least 1); the kept width is the longest length rounded up to a multiple of
    8, capped at S. One device-to-host read (the kept width).

    Args:
        ctx: `[B, S, C]` text embeddings, zero-padded along S.

    Returns:
        `(ctx[:, :keep], seqused int32 [B], ln_pad float32 [B])` with
        ln_pad = log(S - length) (-inf when nothing was padded).
    """
    S = ctx.shape[1]
    index = torch.arange(1, S + 1, device=ctx.device)
    lengths = ((ctx != 0).any(-1) * index).amax(1).clamp_min(1)
    keep = min(S, (int(lengths.max()) + 7) // 8 * 8)
    seqused = lengths.to(torch.int32).contiguous()
    ln_pad = torch.log((S - lengths).float())
    return ctx[:, :keep], seqused, ln_pad


_ELEM_BYTES = {torch.bfloat16: 2, torch.float16: 2, torch.float32: 4}


def context_lengths(ctx: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Key lengths and log padding of a zero-padded text context, on the GPU.

    The same values as `trim_context` (length of item b = 1-based index of its
    last row with a non-zero element, at least 1; ln_pad = log(S - length)),
    computed by one HIP pass over `ctx` with no device-to-host read. The
    context is not trimmed: K/V projected from all S rows go to
    `cross_attention_trimmed` / `Context` with these values, and the masked
    attention reads only the first `seqused[b]` keys, so the result equals
    the reference's trimmed path (model.py:247-254) without its sync.

    Args:
        ctx: `[B, S, C]` bf16, fp16 or fp32 CUDA tensor, last dim contiguous,
            rows 16-byte aligned (C * element size a multiple of 16 bytes).

    Returns:
        `(seqused int32 [B], ln_pad float32 [B])` on ctx's device.
    """
    _check(ctx)
    if ctx.dim() != 3 or ctx.stride(2) != 1:
        raise ValueError("context_lengths: ctx must be [B, S, C] with a contiguous last dim")
    if ctx.dtype not in _ELEM_BYTES:
        raise ValueError(f"context_lengths: unsupported dtype {ctx.dtype}")
    B, S, C = ctx.shape
    if S == 0:
        raise ValueError("context_lengths: empty context (S = 0)")
    seqused = torch.empty(B, dtype=torch.int32, device=ctx.device)
    ln_pad = torch.empty(B, dtype=torch.float32, device=ctx.device)
    ws_bytes = _lib.lib().aa_context_lengths_workspace(B, S)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=ctx.device)
    with torch.cuda.device(ctx.device):
        _lib.check(
            _lib.lib().aa_context_lengths(
                ctx.data_ptr(), B, S, C, ctx.stride(0), ctx.stride(1), _ELEM_BYTES[ctx.dtype],
                seqused.data_ptr(), ln_pad.data_ptr(), ws.data_ptr(), ws_bytes, _lib.stream(ctx),
            ),
            "context_lengths",
        )
    return seqused, ln_pad
