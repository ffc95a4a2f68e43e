"""ctypes binding of libanima_attn.so (declared in include/anima_attn.h).

The library is loaded lazily, after torch, so that it shares torch's HIP
runtime (both link libamdhip64.so.7; the dynamic loader reuses the copy torch
already mapped) and therefore torch's streams and device memory. There is no
fallback: if the library is missing or cannot be loaded, every kernel call
raises RuntimeError.
"""

from __future__ import annotations

import ctypes
import functools
import threading
from ctypes import Structure, c_char_p, c_float, c_int, c_int64, c_size_t, c_void_p
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().with_name("libanima_attn.so")
ABI_VERSION = 3

AA_OK = 0
AA_EINVAL = -1
AA_EUNSUPPORTED = -2
AA_EHIP = -3

DTYPE_CODES = {torch.bfloat16: 0}

# Entry points of include/anima_attn.h with their argument types.
_I64 = c_int64
_PROTOTYPES: dict[str, tuple[object, list[object]]] = {
    "aa_abi_version": (c_int, []),
    "aa_last_error": (c_char_p, []),
    "aa_qkv_norm_rope_fwd": (
        c_int,
        [c_void_p] * 4 + [c_void_p] * 4 + [_I64] * 4 + [c_float, c_int, c_void_p],
    ),
    "aa_proj_head_norm": (
        c_int,
        [c_void_p, _I64, c_void_p, _I64, c_void_p, c_void_p] + [_I64] * 4 + [c_float, c_int, c_void_p],
    ),
    "aa_kv_proj_norm": (
        c_int,
        [c_void_p, _I64, c_void_p, _I64, c_void_p, c_void_p, c_void_p] + [_I64] * 4
        + [c_float, c_int, c_void_p],
    ),
    "aa_qkv_proj_norm_rope": (
        c_int,
        [c_void_p, _I64, c_void_p] + [c_void_p] * 3 + [c_void_p] * 4 + [_I64] * 4
        + [c_float, c_int, c_void_p],
    ),
    "aa_head_norm_fwd": (c_int, [c_void_p] * 3 + [_I64] * 4 + [c_float, c_int, c_void_p]),
    "aa_qkv_norm_rope_bwd_workspace": (c_size_t, [_I64] * 4),
    "aa_qkv_norm_rope_bwd": (
        c_int,
        [c_void_p] * 5 + [c_void_p] * 4 + [c_void_p] * 2 + [c_void_p, c_size_t] + [_I64] * 4
        + [c_float, c_int, c_void_p],
    ),
    "aa_head_norm_bwd_workspace": (c_size_t, [_I64] * 4),
    "aa_head_norm_bwd": (
        c_int,
        [c_void_p] * 5 + [c_void_p, c_size_t] + [_I64] * 4 + [c_float, c_int, c_void_p],
    ),
    "aa_attn_fwd": (c_int, [c_void_p, c_void_p]),
    "aa_attn_fwd_noalloc": (c_int, [c_void_p, c_void_p]),
    "aa_attn_fwd_workspace": (c_size_t, [_I64] * 5),
    "aa_attn_bwd_workspace": (c_size_t, [_I64] * 5),
    "aa_attn_bwd": (c_int, [c_void_p, c_void_p, c_size_t, c_void_p]),
    "aa_ctx_scale_fwd": (c_int, [c_void_p] * 4 + [_I64] * 4 + [c_int, c_void_p]),
    "aa_ctx_scale_bwd": (c_int, [c_void_p] * 6 + [_I64] * 4 + [c_int, c_void_p]),
    "aa_context_lengths_workspace": (c_size_t, [_I64] * 2),
    "aa_rowquant": (c_int, [c_void_p, _I64, _I64, c_int, c_void_p, c_void_p, c_int, c_void_p]),
    "aa_context_lengths": (
        c_int, [c_void_p] + [_I64] * 5 + [c_int] + [c_void_p] * 3 + [c_size_t, c_void_p]
    ),
}

EXPORTED = tuple(_PROTOTYPES)


class AttnFwdArgs(Structure):
    """Mirror of aa_attn_fwd_args."""

    _fields_ = [
        ("q", c_void_p),
        ("k", c_void_p),
        ("v", c_void_p),
        ("out", c_void_p),
        ("lse", c_void_p),
        ("seqused_k", c_void_p),
        ("ln_pad", c_void_p),
        ("q_stride", c_int64 * 3),
        ("k_stride", c_int64 * 3),
        ("v_stride", c_int64 * 3),
        ("out_stride", c_int64 * 3),
        ("B", c_int64),
        ("Sq", c_int64),
        ("Sk", c_int64),
        ("H", c_int64),
        ("hd", c_int64),
        ("softmax_scale", c_float),
        ("dtype", c_int),
        ("workspace", c_void_p),
        ("workspace_bytes", c_size_t),
    ]


class AttnBwdArgs(Structure):
    """Mirror of aa_attn_bwd_args."""

    _fields_ = [
        ("dout", c_void_p),
        ("q", c_void_p),
        ("k", c_void_p),
        ("v", c_void_p),
        ("out", c_void_p),
        ("lse", c_void_p),
        ("dq", c_void_p),
        ("dk", c_void_p),
        ("dv", c_void_p),
        ("dout_stride", c_int64 * 3),
        ("q_stride", c_int64 * 3),
        ("k_stride", c_int64 * 3),
        ("v_stride", c_int64 * 3),
        ("out_stride", c_int64 * 3),
        ("dq_stride", c_int64 * 3),
        ("dk_stride", c_int64 * 3),
        ("dv_stride", c_int64 * 3),
        ("B", c_int64),
        ("Sq", c_int64),
        ("Sk", c_int64),
        ("H", c_int64),
        ("hd", c_int64),
        ("softmax_scale", c_float),
        ("dtype", c_int),
    ]


_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    """The loaded library, with argument types set (raises if missing)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"{LIB_PATH.name} is not built: run `python anima-flat_amd/build.py` "
                    "(or __graft_entry__.build())"
                )
            handle = ctypes.CDLL(str(LIB_PATH))
            for name, (restype, argtypes) in _PROTOTYPES.items():
                fn = getattr(handle, name)
                fn.restype = restype
                fn.argtypes = argtypes
            version = handle.aa_abi_version()
            if version != ABI_VERSION:
                raise RuntimeError(
                    f"{LIB_PATH.name} has ABI version {version}, expected {ABI_VERSION}"
                )
            _lib = handle
    return _lib


def available() -> bool:
    """True if the library loads."""
    try:
        lib()
    except (OSError, RuntimeError):
        return False
    return True


def check(rc: int, what: str) -> None:
    """Map a return code of the library to a Python exception."""
    if rc == AA_OK:
        return
    msg = (lib().aa_last_error() or b"").decode(errors="replace")
    if rc in (AA_EINVAL, AA_EUNSUPPORTED):
        raise ValueError(f"{what}: {msg}")
    raise RuntimeError(f"{what}: {msg} (code {rc})")


def dtype_code(t: torch.Tensor) -> int:
    try:
        return DTYPE_CODES[t.dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {t.dtype}: only bfloat16 is implemented") from None


def on_device(fn):
    """Decorator: runs fn(t, ...) with the GPU of its first argument t as the
    current HIP device. The library reads the current device (its CU count sizes
    the forward's split plan and grid) and launches on the stream it is given,
    which must belong to that same device."""

    @functools.wraps(fn)
    def wrapper(t, *args, **kwargs):
        if not t.is_cuda:  # rejected by fn's own checks
            return fn(t, *args, **kwargs)
        with torch.cuda.device(t.device):
            return fn(t, *args, **kwargs)

    return wrapper


def stream(t: torch.Tensor) -> int:
    """hipStream_t of torch's current stream on t's device."""
    return torch.cuda.current_stream(t.device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def bshd_strides(t: torch.Tensor) -> tuple[int, int, int]:
    """(batch, seq, head) element strides of a [B, S, H, hd] tensor."""
    s = t.stride()
    return (s[0], s[1], s[2])


def c_strides(values: tuple[int, int, int]):
    return (c_int64 * 3)(*values)


def call_attn_fwd(args: AttnFwdArgs, strm: int) -> None:
    check(lib().aa_attn_fwd(ctypes.byref(args), strm), "attn_fwd")


def call_attn_bwd(args: AttnBwdArgs, ws: torch.Tensor | None, ws_bytes: int, strm: int) -> None:
    check(
        lib().aa_attn_bwd(ctypes.byref(args), ptr(ws), ws_bytes, strm),
        "attn_bwd",
    )


__all__ = [
    "AA_EHIP",
    "AA_EINVAL",
    "AA_EUNSUPPORTED",
    "AA_OK",
    "AttnBwdArgs",
    "AttnFwdArgs",
    "EXPORTED",
    "LIB_PATH",
    "available",
    "bshd_strides",
    "c_strides",
    "call_attn_bwd",
    "call_attn_fwd",
    "check",
    "dtype_code",
    "lib",
    "ptr",
    "stream",
]
