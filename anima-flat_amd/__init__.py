"""MI355X (gfx950) attention path of anima-flat's DiT, as hand-written HIP kernels.

Drop-in modules, same public signatures as the reference:
  attention      <- src/attention.py      (use_fa4, attention, cross_attention_trimmed,
                                            ops anima_flat::fa_fwd / fa_fwd_nolse / fa_fwd_k / fa_bwd)
  kernels.rope   <- src/kernels/rope.py   (qkv_norm_rope, head_norm and their ops)
  kernels.ctx_scale <- src/kernels/ctx_scale.py (ctx_scale and its ops)
  kernels.fp8    <- src/kernels/fp8.py    (rowquant and its op: FP8 per-token quantisation of
                                            the attention output)
  context        <- src/model.py:51-119, 247-254 (rope_tables, Context, context trimming,
                                            context_lengths: the trim's lengths on the device)

All compute runs in libanima_attn.so (csrc/, C ABI in include/anima_attn.h),
loaded through ctypes by _lib.py. There is no CPU or SDPA fallback.
"""

from . import _lib  # noqa: F401
from .attention import attention, cross_attention_trimmed, use_fa4  # noqa: F401
from .context import Context, context_lengths, rope_tables, trim_context  # noqa: F401
from .kernels.ctx_scale import ctx_scale  # noqa: F401
from .kernels.fp8 import rowquant  # noqa: F401
from .kernels.rope import head_norm, qkv_norm_rope, qkv_proj_norm_rope  # noqa: F401

__all__ = [
    "Context",
    "attention",
    "context_lengths",
    "cross_attention_trimmed",
    "ctx_scale",
    "head_norm",
    "qkv_norm_rope",
    "qkv_proj_norm_rope",
    "rope_tables",
    "rowquant",
    "trim_context",
    "use_fa4",
]
