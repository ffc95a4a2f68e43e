"""GPU parity of the prologue (QK-RMSNorm + RoPE, head_norm) and ctx_scale kernels."""

from __future__ import annotations

import pytest
import torch

from conftest import parity
from oracle import attn_oracle as ref

pytestmark = pytest.mark.gpu

BF = torch.bfloat16


def _inputs(B, S, H, seed, rope_scale=(1.0, 1.0)):
    return ref.prologue_inputs(B, S, H, 128, seed=seed, rope_scale=rope_scale)


@pytest.mark.parametrize("eps", [1e-6, 1e-5])
@pytest.mark.parametrize("B,S,H,scale", [(1, 1024, 16, (1.0, 1.0)), (2, 4096, 16, (4.0, 4.0)), (3, 7, 3, (1.0, 1.0))])
def test_qkv_norm_rope_forward(pkg, dev, B, S, H, scale, eps):
    inp = _inputs(B, S, H, seed=100 + S, rope_scale=scale)
    with torch.no_grad():
        q, k, v = pkg.qkv_norm_rope(
            inp["qkv"].to(dev, BF), inp["q_weight"].to(dev), inp["k_weight"].to(dev),
            inp["cos"].to(dev), inp["sin"].to(dev), H, eps,
        )
    torch.cuda.synchronize()
    rq, rk, rv = ref.qkv_norm_rope(inp["qkv"], inp["q_weight"], inp["k_weight"], inp["cos"], inp["sin"], H, eps)
    assert q.shape == (B, S, H, 128) and q.dtype == BF
    parity(q, rq, name="q")
    parity(k, rk, name="k")
    assert torch.equal(v.float().cpu(), rv)
    # Bit-level agreement with the bf16-rounded oracle except for rare one-ulp ties.
    mism = (q.float().cpu() != rq).float().mean().item()
    assert mism < 1e-3, f"{mism:.2e} of q elements differ from the rounded oracle"


def test_qkv_norm_rope_grad_variant_copies_v(pkg, dev):
    B, S, H = 1, 64, 4
    inp = _inputs(B, S, H, seed=5)
    qkv = inp["qkv"].to(dev, BF).requires_grad_(True)
    q, k, v = pkg.qkv_norm_rope(qkv, inp["q_weight"].to(dev), inp["k_weight"].to(dev),
                                inp["cos"].to(dev), inp["sin"].to(dev), H, 1e-6)
    torch.cuda.synchronize()
    assert v.is_contiguous() and v.data_ptr() != qkv.data_ptr()
    assert torch.equal(v.detach().float().cpu(), inp["qkv"].view(B, S, 3, H, 128)[:, :, 2])


# Blocks of 64 (token, head) items: 4 whole tokens (H 16), 64 (H 1), blocks
# that straddle tokens (H 3, H 48), and a partial last block.
@pytest.mark.parametrize("B,S,H", [(1, 4096, 16), (2, 50, 3), (1, 333, 1), (1, 77, 48)])
def test_qkv_norm_rope_backward(pkg, dev, B, S, H):
    eps = 1e-6
    inp = _inputs(B, S, H, seed=200 + S)
    qkv = inp["qkv"].to(dev, BF).requires_grad_(True)
    qw = inp["q_weight"].to(dev).requires_grad_(True)
    kw = inp["k_weight"].to(dev).requires_grad_(True)
    q, k, v = pkg.qkv_norm_rope(qkv, qw, kw, inp["cos"].to(dev), inp["sin"].to(dev), H, eps)
    g = torch.Generator().manual_seed(201)
    dq, dk, dv = (ref.bf16_normal((B, S, H, 128), g) for _ in range(3))
    torch.autograd.backward((q, k, v), (dq.to(dev, BF), dk.to(dev, BF), dv.to(dev, BF)))
    torch.cuda.synchronize()
    edqkv, edqw, edkw = ref.qkv_norm_rope_backward(
        inp["qkv"], dq, dk, dv, inp["q_weight"], inp["k_weight"], inp["cos"], inp["sin"], H, eps
    )
    parity(qkv.grad, edqkv, name="dqkv")
    # Weight grads sum B*S*H terms: compare relative to their magnitude.
    tol = 2e-2 * max(1.0, edqw.abs().max().item())
    parity(qw.grad, edqw, max_abs=tol, name="dq_weight")
    parity(kw.grad, edkw, max_abs=2e-2 * max(1.0, edkw.abs().max().item()), name="dk_weight")


@pytest.mark.parametrize("B,S,H", [(1, 4096, 16), (1, 1000, 4), (2, 50, 3)])
def test_qkv_norm_rope_backward_deterministic_c_abi(pkg, dev, B, S, H):
    """Two calls through the C ABI on one (uninitialised) workspace give the
    op's results bit for bit: the weight-gradient reduction sums in a fixed
    order whatever the number of partial records (1024, 63 and 5 blocks of 64
    (token, head) items)."""
    import ctypes

    L = pkg._lib
    lib = L.lib()
    eps = 1e-6
    inp = _inputs(B, S, H, seed=300 + S)
    g = torch.Generator().manual_seed(301)
    qkv = inp["qkv"].to(dev, BF)
    dq, dk, dv = (ref.bf16_normal((B, S, H, 128), g).to(dev, BF) for _ in range(3))
    qw, kw = inp["q_weight"].to(dev), inp["k_weight"].to(dev)
    cos, sin = inp["cos"].to(dev), inp["sin"].to(dev)
    expected = torch.ops.anima_flat.qkv_norm_rope_bwd(qkv, dq, dk, dv, qw, kw, cos, sin, H, eps)
    ws_bytes = lib.aa_qkv_norm_rope_bwd_workspace(B, S, H, 128)
    ws = torch.full((ws_bytes // 4,), float("nan"), dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream().cuda_stream
    for call in range(2):
        dqkv = torch.full_like(qkv, float("nan"))
        dqw = torch.full((128,), float("nan"), device=dev)
        dkw = torch.full((128,), float("nan"), device=dev)
        rc = lib.aa_qkv_norm_rope_bwd(
            qkv.data_ptr(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), dqkv.data_ptr(),
            qw.data_ptr(), kw.data_ptr(), cos.data_ptr(), sin.data_ptr(), dqw.data_ptr(),
            dkw.data_ptr(), ws.data_ptr(), ws_bytes, B, S, H, 128, ctypes.c_float(eps), 0, stream)
        L.check(rc, "qkv_norm_rope_bwd")
        torch.cuda.synchronize()
        assert torch.equal(dqkv, expected[0]), f"call {call}: dqkv"
        assert torch.equal(dqw, expected[1]) and torch.equal(dkw, expected[2]), f"call {call}: weight grads"


@pytest.mark.parametrize("B,S,H", [(2, 4096, 16), (1, 9, 5), (1, 300, 1)])
def test_head_norm_forward_backward(pkg, dev, B, S, H):
    eps = 1e-6
    g = torch.Generator().manual_seed(300 + S)
    x = ref.bf16_normal((B, S, H * 128), g)
    w = ref.norm_weight(128, g)
    xd = x.to(dev, BF).requires_grad_(True)
    wd = w.to(dev).requires_grad_(True)
    y = pkg.head_norm(xd, wd, H, eps)
    dy = ref.bf16_normal((B, S, H, 128), g)
    y.backward(dy.to(dev, BF))
    torch.cuda.synchronize()
    parity(y, ref.head_norm(x, w, H, eps), name="head_norm y")
    edx, edw = ref.head_norm_backward(x, dy, w, H, eps)
    parity(xd.grad, edx, name="head_norm dx")
    parity(wd.grad, edw, max_abs=2e-2 * max(1.0, edw.abs().max().item()), name="head_norm dw")


def test_ctx_scale_forward_backward(pkg, dev):
    B, S, H = 2, 130, 3
    g = torch.Generator().manual_seed(400)
    out = ref.bf16_normal((B, S, H, 128), g)
    lse = torch.randn(B, H, S, generator=g) * 2 + 3
    ln_pad = torch.tensor([float("-inf"), 2.5])
    dy = ref.bf16_normal((B, S, H, 128), g)
    od = out.to(dev, BF).requires_grad_(True)
    ld = lse.to(dev).requires_grad_(True)
    y = pkg.ctx_scale(od, ld, ln_pad.to(dev))
    y.backward(dy.to(dev, BF))
    torch.cuda.synchronize()
    parity(y, ref.ctx_scale(out, lse, ln_pad), name="ctx_scale y")
    edo, edl = ref.ctx_scale_backward(out, lse, ln_pad, dy)
    parity(od.grad, edo, name="ctx_scale dout")
    parity(ld.grad, edl, max_abs=2e-2 * max(1.0, edl.abs().max().item()), name="ctx_scale dlse")
    # ln_pad = -inf: no padding removed, the gain is exactly 1.
    assert torch.equal(y[0].float().cpu(), out[0])
