"""aa_attn_fwd_noalloc (the forward with no allocation) against aa_attn_fwd.

Both entry points are called through the C ABI with the same arguments; the
no-alloc one keeps the key-split partials in the library's fixed per-device
scratch array instead of a caller workspace. Same kernels, so the outputs and
LSE must be bit-identical. Two calls in a row, the second with a smaller
input, both of which use the scratch array (a partial last round of work
items is split over key ranges), then one that needs no partials.
"""

from __future__ import annotations

import ctypes
import math

import pytest
import torch

from oracle import attn_oracle as ref

pytestmark = pytest.mark.gpu

BF = torch.bfloat16
DEV = "cuda:0"


def _args(L, q, k, v, out, lse, seqused, ln_pad):
    a = L.AttnFwdArgs()
    a.q, a.k, a.v, a.out = q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr()
    a.lse = lse.data_ptr()
    a.seqused_k = None if seqused is None else seqused.data_ptr()
    a.ln_pad = None if ln_pad is None else ln_pad.data_ptr()
    for name, t in (("q_stride", q), ("k_stride", k), ("v_stride", v), ("out_stride", out)):
        setattr(a, name, (ctypes.c_int64 * 3)(*t.stride()[:3]))
    a.B, a.Sq, a.Sk, a.H, a.hd = q.shape[0], q.shape[1], k.shape[1], q.shape[2], q.shape[3]
    a.softmax_scale = 1.0 / math.sqrt(q.shape[3])
    a.dtype = 0  # bf16
    return a


def _both(pkg, B, Sq, Sk, H, seed, lens=None, hd=128):
    """(out, lse) of aa_attn_fwd with a torch workspace and of aa_attn_fwd_noalloc."""
    L = pkg._lib
    lib = L.lib()
    g = torch.Generator().manual_seed(seed)
    q, k, v = (ref.bf16_normal((B, S, H, hd), g).to(DEV, BF) for S in (Sq, Sk, Sk))
    seqused = ln_pad = None
    if lens is not None:
        seqused = torch.tensor(lens, dtype=torch.int32, device=DEV)
        ln_pad = torch.log(torch.tensor([float(Sk - n) for n in lens])).to(DEV)
    stream = torch.cuda.current_stream().cuda_stream
    ws_bytes = lib.aa_attn_fwd_workspace(B, Sq, Sk, H, hd)
    results = []
    for noalloc in (False, True):
        out = torch.full((B, Sq, H, hd), float("nan"), dtype=BF, device=DEV)
        lse = torch.full((B, H, Sq), float("nan"), dtype=torch.float32, device=DEV)
        a = _args(L, q, k, v, out, lse, seqused, ln_pad)
        if noalloc:
            rc = lib.aa_attn_fwd_noalloc(ctypes.byref(a), stream)
        else:
            ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=DEV)
            if ws_bytes:
                a.workspace, a.workspace_bytes = ws.data_ptr(), ws_bytes
            rc = lib.aa_attn_fwd(ctypes.byref(a), stream)
        L.check(rc, "attn_fwd_noalloc" if noalloc else "attn_fwd")
        torch.cuda.synchronize()
        results.append((out, lse))
    return ws_bytes, results, (q, k, v)


@pytest.mark.parametrize(
    "B,Sq,Sk,H,lens,split,hd",
    [
        (1, 1024, 1024, 16, None, True, 128),  # config 1: 64 work items, split 4 ways
        (1, 300, 200, 3, [150], True, 128),  # smaller, masked with the padding correction
        (1, 4096, 4096, 16, None, False, 128),  # config 2: one full round, no partials
        # 9216 keys: the first-tile-max form with its fix-up launch, 72 items x 3 key ranges
        (1, 9216, 9216, 2, None, True, 128),
        (1, 16384, 16384, 1, None, True, 384),  # the VAE attention: 128 items x 2 key ranges
        (1, 4096, 4096, 1, None, True, 384),  # smaller again: 32 items x 8 key ranges
    ],
)
def test_noalloc_matches_allocating_entry_point(pkg, B, Sq, Sk, H, lens, split, hd):
    ws_bytes, ((o1, l1), (o2, l2)), (q, k, v) = _both(pkg, B, Sq, Sk, H, seed=900 + Sq, lens=lens, hd=hd)
    assert (ws_bytes > 0) == split
    assert torch.equal(o1, o2), f"out differs at {(o1 != o2).sum().item()} elements"
    assert torch.equal(l1, l2)
    assert not torch.isnan(o2.float()).any()


def test_noalloc_rejects_null_args(pkg):
    L = pkg._lib
    assert L.lib().aa_attn_fwd_noalloc(None, None) == L.AA_EINVAL
