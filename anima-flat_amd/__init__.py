"""MI355X (gfx950) attention path of anima-flat's DiT, as hand-written HIP kernels.

Drop-in modules, same public signatures as the reference:
  attention      <- src/attention.py      (use_fa4, attention, cross_attention_trimmed,
                                            ops anima_flat::fa_fwd / fa_fwd_nolse / fa_fwd_k / fa_bwd)
  kernels.rope   <- src/kernels/rope.py   (qkv_norm_rope, head_norm and their ops)
  kernels.ctx_scale <- src/kernels/ctx_scale.py (ctx_scale and its ops)
  context        <- src/model.py:51-119, 247-254 (rope_tables, Context, context trimming,
                                            context_lengths: the trim's lengths on the device)
  vae            <- the `_attend` of src/vae.py:10-13, 239 (attend: the VAE mid-block attention,
                                            head_dim 384; op anima_flat_amd::attend_d384)

Opt-in modules, not imported here (import them explicitly):
  kernels.fp8    <- rowquant of src/kernels/fp8.py (op anima_flat::rowquant: FP8 per-token
                    quantisation of the attention output). The reference's fp8.py registers the
                    same op name and holds the rest of the FP8 path, so importing this module by
                    default would clash with it.
  kernels.proj   input projections with their normalisation fused (qkv_proj_norm_rope,
                 proj_head_norm, kv_proj_norm; ops anima_flat_amd::qkv_proj_norm_rope /
                 proj_head_norm / kv_proj_norm): the GEMM + norm pairs of src/model.py:308-316,
                 :324 and :256-258 in one kernel each; no single counterpart in the reference.

Every op is registered through kernels.common.custom_op, which raises if the name is already
registered in the process (torch.library would otherwise re-bind it silently). Ops this package
adds beyond the reference's live in the `anima_flat_amd::` namespace.

All compute runs in libanima_attn.so (csrc/, C ABI in include/anima_attn.h),
loaded through ctypes by _lib.py. There is no CPU or SDPA fallback.
"""

from . import _lib, vae  # noqa: F401
from .attention import attention, cross_attention_trimmed, use_fa4  # noqa: F401
from .context import Context, context_lengths, rope_tables, trim_context  # noqa: F401
from .kernels.ctx_scale import ctx_scale  # noqa: F401
from .kernels.rope import head_norm, qkv_norm_rope  # noqa: F401

__all__ = [
    "Context",
    "attention",
    "context_lengths",
    "cross_attention_trimmed",
    "ctx_scale",
    "head_norm",
    "qkv_norm_rope",
    "rope_tables",
    "trim_context",
    "use_fa4",
]
