"""The VAE decoder's mid-block attention (head_dim 384) on MI355X.

Drop-in for `_attend` of anima-flat's src/vae.py:10-13, the attention that
`VAE._attention` (vae.py:230-241) runs on one head of C = 384 channels over the
S = (H/8)(W/8) latent positions (16,384 at 1024x1024): ffpa_attn_func when
ffpa-attn is installed, else torch SDPA. Same call, `attend(q, k, v)` on
`[B, heads, S, 384]` tensors, softmax(q k^T / sqrt(384)) v, non-causal.

The kernel is libanima_attn.so's head-dim-384 forward (aa_attn_fwd with
hd = 384, csrc/attn_fwd_d384.hip). It reads q, k, v in place through their
strides (the [B, S, heads, 384] transposed views), writes a fresh output, and
has no backward: the decoder runs under no_grad (ffpa-attn has none either).
bf16 only.
"""

from __future__ import annotations

import torch

from .attention import _launch_fwd, _prep
from .kernels.common import _check, custom_op

HEAD_DIM = 384


@custom_op("anima_flat_amd::attend_d384", mutates_args=())
def _attend_d384(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """[B, S, H, 384] q, k, v -> [B, S, H, 384] output (contiguous)."""
    out, _ = _launch_fwd(q, k, v, want_lse=False, head_dims=(HEAD_DIM,))
    return out


@_attend_d384.register_fake
def _(q, k, v):
    return torch.empty_like(q, memory_format=torch.contiguous_format)


def attend(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """softmax(q k^T / sqrt(d)) v over the sequence dimension, d = 384.

    Mirrors the call at src/vae.py:239 (`_attend(q, k, v)`, ffpa_attn_func /
    F.scaled_dot_product_attention layout).

    Args:
        q: Queries `[B, heads, Sq, 384]`, bf16, on the GPU.
        k: Keys `[B, heads, Sk, 384]`.
        v: Values `[B, heads, Sk, 384]`.

    Returns:
        `[B, heads, Sq, 384]` in q's dtype (a transposed view of a contiguous
        `[B, Sq, heads, 384]` result).

    Raises:
        ValueError: for CPU tensors, a dtype other than bf16, a head dim other
            than 384 or inconsistent shapes.
        RuntimeError: when gradients are required, or a launch fails.
    """
    _check(q, k, v)
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("q, k, v must be [B, heads, S, 384]")
    if torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad):
        raise RuntimeError("attend (head_dim 384) has no backward: the VAE decoder runs without grad")
    qs, ks, vs = (_prep(t.transpose(1, 2)) for t in (q, k, v))
    return _attend_d384(qs, ks, vs).transpose(1, 2)
