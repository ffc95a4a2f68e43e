"""The path's launches under HIP-graph capture: replays equal the eager results.

bench.py times the short ops as HIP graphs, and a caller may capture the
denoiser step. Every entry point launches only kernels (no memsets, no host
reads, workspaces from the caller), so a captured sequence must reproduce the
eager outputs bit for bit on every replay, with other eager work in between.
"""

from __future__ import annotations

import pytest
import torch

from conftest import parity
from oracle import attn_oracle as ref

pytestmark = pytest.mark.gpu

BF = torch.bfloat16


def test_graph_replays_match_eager(pkg, fp8, proj):
    dev = torch.device("cuda:0")
    B, S, H, d = 2, 512, 4, 128
    inp = ref.prologue_inputs(B, S, H, d, seed=77)
    qkv = inp["qkv"].to(dev, BF)
    qw, kw = inp["q_weight"].to(dev), inp["k_weight"].to(dev)
    cos, sin = inp["cos"].to(dev), inp["sin"].to(dev)
    g = torch.Generator().manual_seed(78)
    x = ref.bf16_normal((B, 300, H * d), g).to(dev, BF)
    w = ref.norm_weight(d, g).to(dev)
    kc = ref.bf16_normal((B, 96, H, d), g).to(dev, BF)
    vc = ref.bf16_normal((B, 96, H, d), g).to(dev, BF)
    ctx = torch.zeros(B, 96, 64, dtype=BF, device=dev)
    ctx[0, :40] = 1.0
    ctx[1, :71] = -2.0
    hid = ref.bf16_normal((B, S, H * d), g).to(dev, BF)
    wqkv = (torch.randn(3 * H * d, H * d, generator=g) * (H * d) ** -0.5).to(dev, BF)

    def step():
        q, k, v = pkg.qkv_norm_rope(qkv, qw, kw, cos, sin, H, 1e-6)
        o_self = pkg.attention(q, k, v)
        qx = pkg.head_norm(x, w, H, 1e-6)
        seq, lnp = pkg.context_lengths(ctx)
        o_cross = pkg.cross_attention_trimmed(qx, kc, vc, seq, lnp)
        oq, os_ = fp8.rowquant(o_self)
        pq, pk, pv = proj.qkv_proj_norm_rope(hid, wqkv, qw, kw, cos, sin, H, 1e-6)
        return [o_self, o_cross, oq.view(torch.uint8), os_, seq, lnp, pq, pk, pv]

    with torch.no_grad():
        eager = [t.clone() for t in step()]
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            step()  # warm the caching allocator on the capture stream
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            outs = step()
        for i in range(3):
            # eager work in between that reuses the same kernels on other data
            pkg.attention(*(ref.bf16_normal((1, 130, 2, d), g).to(dev, BF) for _ in range(3)))
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            for a, e in zip(outs, eager):
                assert torch.equal(a, e), f"replay {i}: {a.dtype} {tuple(a.shape)} differs"


def test_graph_replays_split_backward_and_projections(pkg, proj):
    """The launches the first test leaves out: the key-split forward (64 work
    items of 256 queries on the chip's CUs: partials in a workspace, then the
    combine pass), the backward (dq then dkdv, stats in a workspace), the
    cross-attention projections and the head_dim-384 forward (split as well)."""
    vae = pkg.vae
    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(91)
    d = 128
    q1, k1, v1 = (ref.bf16_normal((1, 1024, 16, d), g).to(dev, BF) for _ in range(3))
    qb, kb, vb = (ref.bf16_normal((1, 320, 2, d), g).to(dev, BF) for _ in range(3))
    dout = ref.bf16_normal((1, 320, 2, d), g).to(dev, BF)
    xq = ref.bf16_normal((2, 200, 512), g).to(dev, BF)
    wq = (torch.randn(4 * d, 512, generator=g) * 512**-0.5).to(dev, BF)
    nw = ref.norm_weight(d, g).to(dev)
    ctx = ref.bf16_normal((2, 77, 256), g).to(dev, BF)
    wkv = (torch.randn(2 * 4 * d, 256, generator=g) * 256**-0.5).to(dev, BF)
    q3, k3, v3 = (ref.bf16_normal((1, 1, 1024, 384), g).to(dev, BF) for _ in range(3))

    def step():
        o1 = torch.ops.anima_flat.fa_fwd_nolse(q1, k1, v1)
        ob, lse = torch.ops.anima_flat.fa_fwd(qb, kb, vb)
        dq, dk, dv = torch.ops.anima_flat.fa_bwd(dout, qb, kb, vb, ob, lse)
        y = proj.proj_head_norm(xq, wq, nw, 4, 1e-6)
        kk, vv = proj.kv_proj_norm(ctx, wkv, nw.to(BF), 4, 1e-6)
        o3 = vae.attend(q3, k3, v3)
        return [o1, ob, lse, dq, dk, dv, y, kk, vv, o3]

    with torch.no_grad():
        eager = [t.clone() for t in step()]
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            step()
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            outs = step()
        for i in range(3):
            # eager launches of the same kernels on other shapes in between
            torch.ops.anima_flat.fa_fwd_nolse(*(ref.bf16_normal((1, 700, 3, d), g).to(dev, BF) for _ in range(3)))
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            for j, (a, e) in enumerate(zip(outs, eager)):
                assert torch.equal(a, e), f"replay {i}: output {j} {a.dtype} {tuple(a.shape)} differs"


def test_graph_replays_first_tile_max_with_fixup(pkg, monkeypatch):
    """The one-wave forward's first-tile-max form (forced) under capture: its two
    launches, on ordinary inputs and on inputs whose later scores overflow the first
    tile's exponent range, so that the captured fix-up launch re-runs marked blocks
    on every replay. Replays equal the eager outputs bit for bit and the oracle."""
    dev = torch.device("cuda:0")
    d = 128
    g = torch.Generator().manual_seed(93)
    q0, k0, v0 = (ref.bf16_normal((1, 512, 2, d), g) for _ in range(3))
    # Spiked: every query gets 60 u, keys 1500 and 3000 become 20 u (u a unit
    # vector): their scores exceed the first tile's max by ~134 in log2 units.
    qs = ref.bf16_normal((1, 300, 2, d), g)
    ks = ref.bf16_normal((1, 3100, 2, d), g)
    vs = ref.bf16_normal((1, 3100, 2, d), g)
    u = torch.randn(d, generator=g)
    u = u / u.norm()
    qs = (qs + 60.0 * u).to(BF).float()
    ks[:, [1500, 3000]] = (20.0 * u).to(BF).float()
    k0 = torch.cat([k0, ref.bf16_normal((1, 4096 - 512, 2, d), g)], dim=1)
    v0 = torch.cat([v0, ref.bf16_normal((1, 4096 - 512, 2, d), g)], dim=1)
    args0 = [t.to(dev, BF) for t in (q0, k0, v0)]
    args1 = [t.to(dev, BF) for t in (qs, ks, vs)]
    monkeypatch.setenv("AA_FWD_KERNEL", "1w")
    monkeypatch.setenv("AA_FWD_FIRST_TILE_MAX", "1")

    def step():
        o0, l0 = torch.ops.anima_flat.fa_fwd(*args0)
        o1, l1 = torch.ops.anima_flat.fa_fwd(*args1)
        return [o0, l0, o1, l1]

    with torch.no_grad():
        eager = [t.clone() for t in step()]
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            step()
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            outs = step()
        for i in range(3):
            torch.ops.anima_flat.fa_fwd_nolse(*(ref.bf16_normal((1, 700, 3, d), g).to(dev, BF) for _ in range(3)))
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            for j, (a, e) in enumerate(zip(outs, eager)):
                assert torch.equal(a, e), f"replay {i}: output {j} {a.dtype} {tuple(a.shape)} differs"
    monkeypatch.delenv("AA_FWD_KERNEL")
    monkeypatch.delenv("AA_FWD_FIRST_TILE_MAX")
    parity(eager[0], ref.attention_lse(q0, k0, v0)[0], name="first-tile max, ordinary rows")
    parity(eager[2], ref.attention_lse(qs, ks, vs)[0], name="first-tile max, fixed-up rows")
