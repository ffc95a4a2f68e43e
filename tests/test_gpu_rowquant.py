"""GPU parity of the FP8 row quantisation (aa_rowquant) against the CPU oracle.

Without GELU the result is integer-exact: the same scales (float32 bits) and
the same e4m3fn bytes as the oracle (IEEE division, round to nearest even).
With GELU the device exp differs from the CPU's by an ulp now and then, so a
few bytes may land on the neighbouring e4m3fn value.
"""

from __future__ import annotations

import pytest
import torch

from oracle import attn_oracle as ref

pytestmark = pytest.mark.gpu


def _rows(B, S, K, seed, spread=False):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, S, K, generator=g)
    if spread:  # magnitudes over 2^-20 .. 2^10: many values land in the subnormal range
        x = x * torch.exp2(torch.randint(-20, 11, (B, S, K), generator=g).float())
    return x.to(torch.bfloat16)


@pytest.mark.parametrize(
    "B,S,K,spread",
    [
        (2, 64, 2048, False),  # attention output rows (H * hd = 2048)
        (1, 33, 8192, False),  # MLP width, four chunks per lane
        (3, 5, 8, False),  # one chunk per row
        (2, 40, 2048, True),
        (1, 7, 1000, True),  # K not a multiple of 256 * 8
        # Each (units per lane, values per unit) instantiation: 16-value units
        # when K % 16 == 0, 8-value units otherwise.
        (1, 9, 4096, True),
        (1, 5, 3000, False),
        (1, 3, 8184, True),
    ],
)
def test_rowquant_bit_exact(pkg, fp8, B, S, K, spread):
    x = _rows(B, S, K, seed=B * 31 + S + K, spread=spread)
    x[0, 0] = 0.0  # an all-zero row: scale 1e-12 / 448, bytes 0
    q, s = fp8.rowquant(x.to("cuda:0"))
    torch.cuda.synchronize()
    eq, es = ref.rowquant(x)
    assert q.dtype == torch.float8_e4m3fn and q.shape == x.shape and s.shape == (B * S, 1)
    assert torch.equal(s.cpu(), es), (s.cpu() - es).abs().max()
    qb, eb = q.cpu().view(torch.uint8), eq.view(torch.uint8)
    assert torch.equal(qb, eb), f"{(qb != eb).sum().item()} bytes differ"


@pytest.mark.parametrize("K", [8192, 1000])
def test_rowquant_gelu(pkg, fp8, K):
    B, S = 2, 48
    x = _rows(B, S, K, seed=9) * 3
    q, s = fp8.rowquant(x.to("cuda:0"), gelu=True)
    torch.cuda.synchronize()
    eq, es = ref.rowquant(x, gelu=True)
    torch.testing.assert_close(s.cpu(), es, rtol=4e-7, atol=0)
    a, e = q.cpu().float(), eq.float()
    diff = a != e
    assert diff.float().mean().item() < 1e-3, diff.float().mean().item()
    # a differing byte is the neighbouring e4m3fn value: within one e4m3 step (2^-3 relative)
    assert ((a - e).abs() <= e.abs() * 0.1251 + 2.0**-9).all()


def test_rowquant_of_attention_output(pkg, fp8):
    """rowquant(attention(...)) as the model's FP8 path calls it (model.py:446)."""
    g = torch.Generator().manual_seed(13)
    q, k, v = (ref.bf16_normal((1, 256, 16, 128), g) for _ in range(3))
    out = pkg.attention(*(t.to("cuda:0", torch.bfloat16) for t in (q, k, v)))
    oq, os_ = fp8.rowquant(out)
    torch.cuda.synchronize()
    eq, es = ref.rowquant(out.cpu())
    assert torch.equal(os_.cpu(), es) and torch.equal(oq.cpu().view(torch.uint8), eq.view(torch.uint8))


def test_rowquant_every_e4m3_tie_point(pkg, fp8):
    """Every rounding boundary of e4m3fn: each tie point between adjacent codes and its
    neighbouring fp32 values, both signs, through the kernel with scale exactly 1 (each row
    holds 448). Inputs are bf16, so the tie points are exact and the neighbours are the
    adjacent bf16 values."""
    codes = torch.arange(0, 127, dtype=torch.uint8).view(torch.float8_e4m3fn).float()
    ties = (codes[:-1] + codes[1:]) / 2  # exact in bf16 (at most 5 significant bits)
    tb = ties.to(torch.bfloat16)
    assert torch.equal(tb.float(), ties)
    up = torch.nextafter(tb, torch.tensor(1e4, dtype=torch.bfloat16))
    down = torch.nextafter(tb, torch.tensor(0.0, dtype=torch.bfloat16))
    vals = torch.cat([codes.to(torch.bfloat16), tb, up, down])
    vals = torch.cat([vals, -vals])
    K = 128
    n = vals.numel()
    rows = (n + K - 2) // (K - 1)
    x = torch.zeros(rows * (K - 1), dtype=torch.bfloat16)
    x[:n] = vals
    x = torch.cat([torch.full((rows, 1), 448.0, dtype=torch.bfloat16), x.view(rows, K - 1)], 1)
    x = x.view(1, rows, K)
    q, s = fp8.rowquant(x.to("cuda:0"))
    torch.cuda.synchronize()
    eq, es = ref.rowquant(x)
    assert (es == 1.0).all() and torch.equal(s.cpu(), es)
    assert torch.equal(q.cpu().view(torch.uint8), eq.view(torch.uint8))
