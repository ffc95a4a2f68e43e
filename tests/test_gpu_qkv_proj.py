"""GPU parity of the fused QKV projection + prologue (aa_qkv_proj_norm_rope).

Reference: q, k, v = qkv_norm_rope(b.qkv(hid), ...) (src/model.py:308-316),
restated by oracle.qkv_proj_norm_rope (float32 GEMM of the bf16 inputs, rounded
to bf16, then the prologue). The kernel accumulates the GEMM in a different
order, so a projection value near a bf16 rounding boundary can round the other
way, and that one-ulp flip of the input carries through the normalisation as
about one ulp of the output. Outputs are held to rel-L2 5e-3 and a max-abs bar
of max(2e-2, 2^-7 max|expected|) (normalised q, k reach |4..8|, where one bf16
ulp is 0.016..0.03); v, the projection output itself, to one bf16 ulp on
nearly every element.
"""

from __future__ import annotations

import pytest
import torch

from conftest import parity
from oracle import attn_oracle as ref

pytestmark = pytest.mark.gpu

BF = torch.bfloat16


def _inputs(B, S, H, seed, rope_scale=(1.0, 1.0)):
    g = torch.Generator().manual_seed(seed)
    D = H * 128
    hid = ref.bf16_normal((B, S, D), g)
    w = (torch.randn(3 * D, D, generator=g) * D**-0.5).to(BF)
    qw, kw = ref.norm_weight(128, g), ref.norm_weight(128, g)
    h = 1
    while h * h < S:
        h += 1
    cos, sin = ref.rope_tables(h, h, 128, rope_scale)
    return hid, w, qw, kw, cos[:S].contiguous(), sin[:S].contiguous()


def _run(proj, hid, w, qw, kw, cos, sin, H, eps, dev="cuda:0"):
    with torch.no_grad():
        out = proj.qkv_proj_norm_rope(
            hid.to(dev, BF), w.to(dev, BF), qw.to(dev), kw.to(dev), cos.to(dev), sin.to(dev), H, eps
        )
    torch.cuda.synchronize()
    return out


def _check(outs, exps, tag):
    for name, a, e in zip("qkv", outs, exps):
        assert a.dtype == BF and a.is_contiguous() and a.shape == e.shape
        bar = max(2e-2, e.float().abs().max().item() * 2.0**-7)
        parity(a, e.float(), max_abs=bar, name=f"{tag} {name}")
    v, ev = outs[2].float().cpu(), exps[2].float()
    ulp = (v - ev).abs() <= ev.abs() * 2.0**-7 + 1e-30
    assert ulp.float().mean().item() > 0.999, f"{tag}: v beyond one bf16 ulp on {(~ulp).sum().item()} elements"


@pytest.mark.parametrize(
    "B,S,H,eps,scale",
    [
        (1, 4096, 16, 1e-6, (1.0, 1.0)),  # config 2
        (2, 300, 16, 1e-5, (4.0, 4.0)),  # token count not a multiple of 256
        (1, 77, 2, 1e-6, (1.0, 1.0)),  # small H: K = 256, one token tile
        (3, 5, 1, 1e-6, (1.0, 1.0)),
    ],
)
def test_qkv_proj_matches_oracle(pkg, proj, B, S, H, eps, scale):
    hid, w, qw, kw, cos, sin = _inputs(B, S, H, seed=900 + S + H, rope_scale=scale)
    outs = _run(proj, hid, w, qw, kw, cos, sin, H, eps)
    exps = ref.qkv_proj_norm_rope(hid, w, qw, kw, cos, sin, H, eps)
    _check(outs, exps, f"B{B} S{S} H{H}")


def test_qkv_proj_strided_rows_and_equals_unfused_path(pkg, proj):
    """hid as a strided view (row stride 2560 > 2048); the fused result equals
    F.linear + qkv_norm_rope on the GPU to the same bar."""
    B, S, H = 2, 512, 16
    hid, w, qw, kw, cos, sin = _inputs(B, S, H, seed=77)
    wide = torch.zeros(B, S, 2560, dtype=BF)
    wide[:, :, 256:2304] = hid
    dev = "cuda:0"
    view = wide.to(dev)[:, :, 256:2304]
    outs = _run(proj, view, w, qw, kw, cos, sin, H, 1e-6)
    exps = ref.qkv_proj_norm_rope(hid, w, qw, kw, cos, sin, H, 1e-6)
    _check(outs, exps, "strided")
    with torch.no_grad():
        qkv = torch.nn.functional.linear(hid.to(dev, BF), w.to(dev, BF))
        uq, uk, uv = pkg.qkv_norm_rope(qkv, qw.to(dev), kw.to(dev), cos.to(dev), sin.to(dev), H, 1e-6)
    torch.cuda.synchronize()
    for name, a, e in zip("qkv", outs, (uq, uk, uv)):
        bar = max(2e-2, e.float().abs().max().item() * 2.0**-7)
        parity(a, e.float().cpu(), max_abs=bar, name=f"fused vs unfused {name}")


def test_qkv_proj_rejects_bad_inputs(pkg, proj):
    dev = "cuda:0"
    hid = torch.zeros(1, 8, 256, dtype=BF, device=dev)
    w = torch.zeros(768, 256, dtype=BF, device=dev)
    qw = torch.ones(128, device=dev)
    cs = torch.zeros(8, 64, device=dev)
    with pytest.raises(ValueError, match="weight"):
        proj.qkv_proj_norm_rope(hid, w[:, :128], qw, qw, cs, cs, 2)
    with pytest.raises(ValueError, match="hid"):
        proj.qkv_proj_norm_rope(hid[:, :, :128], w, qw, qw, cs, cs, 2)
    with pytest.raises(RuntimeError, match="backward"):
        proj.qkv_proj_norm_rope(hid.clone().requires_grad_(True), w, qw, qw, cs, cs, 2)


def test_qkv_proj_deterministic(pkg, proj):
    hid, w, qw, kw, cos, sin = _inputs(1, 700, 16, seed=31)
    a = _run(proj, hid, w, qw, kw, cos, sin, 16, 1e-6)
    b = _run(proj, hid, w, qw, kw, cos, sin, 16, 1e-6)
    for x, y in zip(a, b):
        assert torch.equal(x, y)
