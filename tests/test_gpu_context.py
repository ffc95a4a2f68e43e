"""GPU checks of the on-device context-length bookkeeping (aa_context_lengths).

Lengths are integer work: bit-exact against the CPU oracle (model.py:248-253).
ln_pad is log of an integer in float32: within 1 ulp of torch's CPU log.
The end-to-end case checks that masked attention over the untrimmed K/V with
these values equals attention over the zero-padded context, to the attention
parity bar.
"""

from __future__ import annotations

import pytest
import torch

from conftest import parity
from oracle import attn_oracle as ref

pytestmark = pytest.mark.gpu


def _padded_context(B, S, C, lengths, g, dtype):
    ctx = torch.zeros(B, S, C)
    for b, n in enumerate(lengths):
        if n > 0:
            ctx[b, :n] = torch.randn(n, C, generator=g)
            ctx[b, n - 1, 0] = 1.0  # the last kept row is non-zero for sure
    return ctx.to(dtype)


def _check(pkg, ctx_cpu, dev="cuda:0"):
    seq, lnp = pkg.context_lengths(ctx_cpu.to(dev))
    torch.cuda.synchronize()
    eseq, elnp = ref.context_lengths(ctx_cpu.float())
    assert seq.dtype == torch.int32 and lnp.dtype == torch.float32
    assert torch.equal(seq.cpu(), eseq), (seq.cpu().tolist(), eseq.tolist())
    torch.testing.assert_close(lnp.cpu(), elnp, rtol=2e-7, atol=0.0)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize(
    "B,S,C,lengths",
    [
        (2, 512, 1024, [58, 322]),  # config 3 lengths
        (3, 77, 64, [0, 77, 31]),  # all padding, no padding; S not a multiple of 32
        (4, 33, 8, [32, 33, 1, 2]),  # rows of 16 / 32 bytes
        (1, 1, 16, [1]),
    ],
)
def test_context_lengths_match_oracle(pkg, dtype, B, S, C, lengths):
    g = torch.Generator().manual_seed(7 + S + C)
    _check(pkg, _padded_context(B, S, C, lengths, g, dtype))


def test_context_lengths_interior_zeros_signed_zero_and_nan(pkg):
    ctx = torch.zeros(3, 64, 16)
    ctx[0, :40] = 1.0
    ctx[0, 5:30] = 0.0  # interior zero rows
    ctx[1, 50, 15] = -0.0  # negative zero only: still all zero -> length 1
    ctx[2, 63, 3] = float("nan")  # NaN counts as non-zero
    for dtype in (torch.bfloat16, torch.float32):
        _check(pkg, ctx.to(dtype))


def test_context_lengths_strided_view(pkg):
    g = torch.Generator().manual_seed(3)
    base = _padded_context(2, 96, 256, [17, 90], g, torch.bfloat16)
    wide = torch.zeros(2, 96, 384, dtype=torch.bfloat16)
    wide[:, :, 64:320] = base
    view = wide.to("cuda:0")[:, :, 64:320]  # row stride 384 elements, offset 128 B
    seq, lnp = pkg.context_lengths(view)
    torch.cuda.synchronize()
    eseq, elnp = ref.context_lengths(base.float())
    assert torch.equal(seq.cpu(), eseq)
    torch.testing.assert_close(lnp.cpu(), elnp, rtol=2e-7, atol=0.0)


def test_context_lengths_rejects_unaligned_rows(pkg):
    with pytest.raises(ValueError, match="16"):
        pkg.context_lengths(torch.zeros(1, 8, 12, dtype=torch.bfloat16, device="cuda:0"))


def test_untrimmed_kv_with_device_lengths_equals_padded_attention(pkg):
    """K/V from the whole padded context + on-device lengths == attention over the padding."""
    B, Sq, H, S_full, C = 2, 256, 4, 96, 64
    g = torch.Generator().manual_seed(51)
    ctx = _padded_context(B, S_full, C, [29, 70], g, torch.bfloat16)
    q = ref.bf16_normal((B, Sq, H, 128), g)
    # K/V rows follow the context: zero where the context row is zero (no bias).
    rows = (ctx != 0).any(-1)[:, :, None, None].float()
    k = ref.bf16_normal((B, S_full, H, 128), g) * rows
    v = ref.bf16_normal((B, S_full, H, 128), g) * rows
    seq, lnp = pkg.context_lengths(ctx.to("cuda:0"))
    dev = [t.to("cuda:0", torch.bfloat16) for t in (q, k, v)]
    out = pkg.cross_attention_trimmed(*dev, seq, lnp)
    torch.cuda.synchronize()
    padded = ref.attention_sdpa(q, k, v).reshape(B, Sq, H * 128)
    parity(out, padded, name="device lengths, untrimmed K/V vs padded")
