"""GPU parity of the fused QKV projection + prologue (aa_qkv_proj_norm_rope).

Reference: q, k, v = qkv_norm_rope(b.qkv(hid), ...) (src/model.py:308-316),
restated by oracle.qkv_proj_norm_rope (float32 GEMM of the bf16 inputs, rounded
to bf16, then the prologue). The kernel accumulates the GEMM in a different
order, so a projection value near a bf16 rounding boundary can round the other
way, and that one-ulp flip of the input carries through the normalisation as
about one ulp of the output. Normalised outputs are held to rel-L2 5e-3 and to
max-abs 2e-2 on all but at most 0.1% of their elements; each of those few may
be off by at most 2e-2 plus one bf16 ulp of its own value (normalised q, k
reach |4..8|, where one ulp is 0.016..0.03). v, the projection output itself,
is held to one bf16 ulp on nearly every element.
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


MAX_FRAC_PAST_BAR = 1e-3  # elements allowed past max-abs 2e-2 (each within one more ulp)


def _normed_parity(a, e, tag):
    """rel-L2 5e-3; |a - e| <= 2e-2 on all but MAX_FRAC_PAST_BAR of the elements;
    every element within 2e-2 + one bf16 ulp of its expected value."""
    af, ef = a.detach().float().cpu(), e.detach().float().cpu()
    assert torch.isfinite(af).all(), f"{tag}: non-finite values"
    err = (af - ef).abs()
    rl = ((af - ef).norm() / ef.norm().clamp_min(1e-30)).item()
    past = (err > 2e-2).float().mean().item()
    worst = (err - (2e-2 + ef.abs() * 2.0**-7)).max().item()
    print(f"[parity] {tag}: max_abs={err.max().item():.3e} rel_l2={rl:.3e} past_2e-2={past:.2e}", flush=True)
    assert rl <= 5e-3, f"{tag}: rel_l2 {rl:.3e} > 5e-3"
    assert past <= MAX_FRAC_PAST_BAR, f"{tag}: {past:.2e} of elements past max-abs 2e-2"
    assert worst <= 0, f"{tag}: an element is off by more than 2e-2 + one bf16 ulp"


def _check(outs, exps, tag):
    for name, a, e in zip("qkv", outs, exps):
        assert a.dtype == BF and a.is_contiguous() and a.shape == e.shape
        if name == "v":
            parity(a, e.float(), name=f"{tag} {name}")
        else:
            _normed_parity(a, e, f"{tag} {name}")
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
        _normed_parity(a, e, f"fused vs unfused {name}")


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


# ------------------------------------------- cross-attention projections --
# proj_head_norm: q = head_norm(b.xq(hid), b.xq_norm, heads, eps) (src/model.py:324).
# kv_proj_norm: k, v = b.xkv(ctx).view(B, S, 2, H, hd).unbind(2); k = F.rms_norm(k, ...)
# (src/model.py:256-258). Oracle: oracle.proj_head_norm / oracle.kv_proj_norm; the
# same bar as above (normalised outputs: _normed_parity; the plain projection v to
# one bf16 ulp on nearly every element).


def _lin_inputs(B, S, K, N, seed):
    g = torch.Generator().manual_seed(seed)
    x = ref.bf16_normal((B, S, K), g)
    w = (torch.randn(N, K, generator=g) * K**-0.5).to(BF)
    return x, w, ref.norm_weight(128, g)


def _normed(a, e, tag):
    assert a.dtype == BF and a.is_contiguous() and a.shape == e.shape
    _normed_parity(a, e, tag)


@pytest.mark.parametrize(
    "B,S,H,K,eps",
    [
        (2, 4096, 16, 2048, 1e-6),  # config 3's query side
        (1, 300, 3, 2048, 1e-5),  # odd head count: half-empty last column pair
        (3, 5, 1, 96, 1e-6),  # K = 96: three k-steps, one head
        (1, 257, 8, 1024, 1e-6),  # K != heads * head_dim
    ],
)
def test_proj_head_norm_matches_oracle(pkg, proj, B, S, H, K, eps):
    x, w, nw = _lin_inputs(B, S, K, H * 128, seed=1300 + S + H)
    with torch.no_grad():
        y = proj.proj_head_norm(x.to("cuda:0", BF), w.to("cuda:0"), nw.to("cuda:0"), H, eps)
    torch.cuda.synchronize()
    _normed(y, ref.proj_head_norm(x, w, nw, H, eps), f"proj_head_norm B{B} S{S} H{H} K{K}")


def test_proj_head_norm_strided_equals_unfused(pkg, proj):
    """x as a strided view; the fused result equals F.linear + head_norm on the GPU."""
    B, S, H, K = 2, 512, 16, 2048
    x, w, nw = _lin_inputs(B, S, K, H * 128, seed=1401)
    dev = "cuda:0"
    wide = torch.zeros(B, S, K + 512, dtype=BF)
    wide[:, :, 128 : 128 + K] = x
    view = wide.to(dev)[:, :, 128 : 128 + K]
    with torch.no_grad():
        y = proj.proj_head_norm(view, w.to(dev), nw.to(dev), H, 1e-6)
        u = pkg.head_norm(torch.nn.functional.linear(x.to(dev, BF), w.to(dev)), nw.to(dev), H, 1e-6)
    torch.cuda.synchronize()
    _normed(y, ref.proj_head_norm(x, w, nw, H, 1e-6), "proj_head_norm strided")
    _normed(y, u.float().cpu(), "proj_head_norm fused vs unfused")


@pytest.mark.parametrize(
    "B,S,H,K,eps",
    [
        (2, 512, 16, 1024, 1e-6),  # config 3's context: text_dim 1024, 512 tokens
        (1, 77, 1, 1024, 1e-5),  # one head: two sections, one column pair
        (3, 40, 5, 256, 1e-6),
    ],
)
def test_kv_proj_norm_matches_oracle(pkg, proj, B, S, H, K, eps):
    ctx, w, kw = _lin_inputs(B, S, K, 2 * H * 128, seed=1500 + S + H)
    kw16 = kw.to(BF)  # the reference passes b.xk_norm.to(k.dtype)
    with torch.no_grad():
        k, v = proj.kv_proj_norm(ctx.to("cuda:0", BF), w.to("cuda:0"), kw16.to("cuda:0"), H, eps)
    torch.cuda.synchronize()
    ek, ev = ref.kv_proj_norm(ctx, w, kw16, H, eps)
    _normed(k, ek, f"kv_proj_norm k B{B} S{S} H{H}")
    assert v.dtype == BF and v.is_contiguous() and v.shape == ev.shape
    vc = v.float().cpu()
    ulp = (vc - ev).abs() <= ev.abs() * 2.0**-7 + 1e-30
    assert ulp.float().mean().item() > 0.999, f"v beyond one bf16 ulp on {(~ulp).sum().item()} elements"


def test_kv_proj_norm_equals_reference_expression(pkg, proj):
    """Against the reference's own torch expression run on the GPU (F.linear, view,
    unbind, F.rms_norm with the weight in the activation dtype), on a strided context."""
    B, S, H, K = 2, 512, 16, 1024
    ctx, w, kw = _lin_inputs(B, S, K, 2 * H * 128, seed=1601)
    dev = "cuda:0"
    wide = torch.zeros(B, S, K + 64, dtype=BF)
    wide[:, :, :K] = ctx
    view = wide.to(dev)[:, :, :K]
    kwd = kw.to(dev)
    with torch.no_grad():
        k, v = proj.kv_proj_norm(view, w.to(dev), kwd.to(BF), H, 1e-6)
        uk, uv = torch.nn.functional.linear(ctx.to(dev, BF), w.to(dev)).view(B, S, 2, H, 128).unbind(2)
        uk = torch.nn.functional.rms_norm(uk, (128,), kwd.to(uk.dtype), 1e-6)
    torch.cuda.synchronize()
    _normed(k, uk.float().cpu(), "kv_proj_norm k vs torch")
    _normed(v, uv.float().cpu(), "kv_proj_norm v vs torch")


@pytest.mark.parametrize("lens", [(58, 322), (200,), (512, 9)])
def test_cross_projections_on_trimmed_context(pkg, proj, lens):
    """trim_context's output (src/model.py:248-253) fed to kv_proj_norm, as
    encode_context does (model.py:256-258): ctx[:, :keep] is a view whose batch
    stride is S * K, not keep * K. Also proj_head_norm on a batch-strided view."""
    B, S, H, K = len(lens), 512, 16, 1024
    ctx, w, kw = _lin_inputs(B, S, K, 2 * H * 128, seed=1650 + sum(lens))
    for b, n in enumerate(lens):
        ctx[b, n:] = 0
    dev = "cuda:0"
    trimmed, seqused, _ = pkg.trim_context(ctx.to(dev, BF))
    keep = trimmed.shape[1]
    assert keep == min(S, (max(lens) + 7) // 8 * 8)
    if B > 1 and keep < S:
        assert trimmed.stride(0) == S * K and not trimmed.is_contiguous()
    kw16 = kw.to(BF)
    with torch.no_grad():
        k, v = proj.kv_proj_norm(trimmed, w.to(dev), kw16.to(dev), H, 1e-6)
    torch.cuda.synchronize()
    assert torch.equal(seqused.cpu(), torch.tensor(lens, dtype=torch.int32))
    ek, ev = ref.kv_proj_norm(ctx[:, :keep], w, kw16, H, 1e-6)
    _normed(k, ek, f"kv_proj_norm on trimmed ctx lens={lens}")
    vc = v.float().cpu()
    ulp = (vc - ev).abs() <= ev.abs() * 2.0**-7 + 1e-30
    assert ulp.float().mean().item() > 0.999, f"v beyond one bf16 ulp on {(~ulp).sum().item()} elements"
    # The query side on a batch-strided view (every other item of a larger batch).
    xq, wq, nq = _lin_inputs(2 * B, 300, 2048, H * 128, seed=1660 + sum(lens))
    with torch.no_grad():
        y = proj.proj_head_norm(xq.to(dev, BF)[::2], wq.to(dev), nq.to(dev), H, 1e-6)
    torch.cuda.synchronize()
    _normed(y, ref.proj_head_norm(xq[::2], wq, nq, H, 1e-6), f"proj_head_norm batch-strided lens={lens}")


def test_cross_projections_reject_bad_inputs(pkg, proj):
    dev = "cuda:0"
    x = torch.zeros(1, 8, 256, dtype=BF, device=dev)
    nw = torch.ones(128, device=dev)
    with pytest.raises(ValueError, match="weight"):
        proj.proj_head_norm(x, torch.zeros(256, 128, dtype=BF, device=dev), nw, 2)
    with pytest.raises(ValueError, match="weight"):
        proj.kv_proj_norm(x, torch.zeros(256, 256, dtype=BF, device=dev), nw, 2)
    with pytest.raises(ValueError, match="head_dim"):
        proj.proj_head_norm(x, torch.zeros(128, 256, dtype=BF, device=dev), nw[:64], 2)
    w = torch.zeros(256, 256, dtype=BF, device=dev)
    with pytest.raises(RuntimeError, match="backward"):
        proj.proj_head_norm(x.clone().requires_grad_(True), w, nw, 2)
    with pytest.raises(RuntimeError, match="backward"):
        proj.kv_proj_norm(x.clone().requires_grad_(True), torch.zeros(512, 256, dtype=BF, device=dev), nw, 2)


# ---------------------------------------------------------- tile shapes --
# The launcher picks one of three workgroup tiles (256 tokens x 2 sections,
# 256 x 3, 128 x 1) by how evenly the workgroups fill the chip; AA_PROJ_TILE
# forces one. Every shape accumulates each output in the same order, so the
# results must be bit-identical; the default shape is held to the oracle above.


def _all_tiles(monkeypatch, fn):
    outs = {}
    for t in "abc":
        monkeypatch.setenv("AA_PROJ_TILE", t)
        with torch.no_grad():
            r = fn()
        torch.cuda.synchronize()
        outs[t] = r if isinstance(r, tuple) else (r,)
    monkeypatch.delenv("AA_PROJ_TILE")
    return outs


def _same_bits(outs, tag):
    for t in "bc":
        for i, (x, y) in enumerate(zip(outs["a"], outs[t])):
            assert torch.equal(x, y), f"{tag}: tile {t} output {i} differs from tile a"


@pytest.mark.parametrize("B,S,H", [(1, 4096, 16), (2, 300, 16), (1, 77, 2), (3, 5, 1), (1, 1100, 5)])
def test_qkv_proj_tile_shapes_identical(pkg, proj, monkeypatch, B, S, H):
    hid, w, qw, kw, cos, sin = _inputs(B, S, H, seed=1700 + S + H)
    dev = "cuda:0"
    args = (hid.to(dev, BF), w.to(dev, BF), qw.to(dev), kw.to(dev), cos.to(dev), sin.to(dev), H, 1e-6)
    outs = _all_tiles(monkeypatch, lambda: proj.qkv_proj_norm_rope(*args))
    _same_bits(outs, f"qkv B{B} S{S} H{H}")
    _check(outs["b"], ref.qkv_proj_norm_rope(hid, w, qw, kw, cos, sin, H, 1e-6), f"tile b B{B} S{S} H{H}")


@pytest.mark.parametrize("B,S,H,K", [(2, 1000, 3, 512), (1, 257, 16, 2048), (1, 31, 1, 64)])
def test_cross_proj_tile_shapes_identical(pkg, proj, monkeypatch, B, S, H, K):
    dev = "cuda:0"
    x, wq, nw = _lin_inputs(B, S, K, H * 128, seed=1800 + S)
    _, wkv, _ = _lin_inputs(B, S, K, 2 * H * 128, seed=1900 + S)
    xd, wqd, wkvd, nwd = x.to(dev, BF), wq.to(dev), wkv.to(dev), nw.to(dev)
    outs = _all_tiles(monkeypatch, lambda: proj.proj_head_norm(xd, wqd, nwd, H, 1e-6))
    _same_bits(outs, f"xq B{B} S{S} H{H} K{K}")
    _normed(outs["c"][0], ref.proj_head_norm(x, wq, nw, H, 1e-6), f"xq tile c B{B} S{S} H{H}")
    outs = _all_tiles(monkeypatch, lambda: proj.kv_proj_norm(xd, wkvd, nwd.to(BF), H, 1e-6))
    _same_bits(outs, f"xkv B{B} S{S} H{H} K{K}")
    ek, _ = ref.kv_proj_norm(x, wkv, nw.to(BF), H, 1e-6)
    _normed(outs["b"][0], ek, f"xkv tile b B{B} S{S} H{H}")


def test_proj_tile_env_rejects_unknown_value(pkg, proj, monkeypatch):
    dev = "cuda:0"
    x = torch.zeros(1, 8, 256, dtype=BF, device=dev)
    monkeypatch.setenv("AA_PROJ_TILE", "z")
    with pytest.raises(ValueError, match="AA_PROJ_TILE"):
        proj.proj_head_norm(x, torch.zeros(256, 256, dtype=BF, device=dev), torch.ones(128, device=dev), 2)
