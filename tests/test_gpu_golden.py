"""HIP kernels against the committed float64 golden vectors (tests/golden/*.npz)."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from conftest import parity

pytestmark = pytest.mark.gpu

GOLD = Path(__file__).resolve().parent / "golden"
BF = torch.bfloat16


def _bits(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy((a.astype(np.uint32) << 16).view(np.float32).copy())


def _g(name):
    return np.load(GOLD / name, allow_pickle=False)


def _dev(t, dtype=BF):
    return t.to("cuda", dtype)


def test_golden_attention(pkg):
    g = _g("attn_small.npz")
    q, k, v = (_dev(_bits(g[n])) for n in ("q", "k", "v"))
    out, lse = torch.ops.anima_flat.fa_fwd(q, k, v)
    torch.cuda.synchronize()
    parity(out, torch.from_numpy(g["out"]), name="golden attention out")
    parity(lse, torch.from_numpy(g["lse"]), max_abs=2e-3, rel_l2=2e-4, name="golden attention lse")


def test_golden_masked_and_trimmed(pkg):
    g = _g("masked_small.npz")
    q, k, v = (_dev(_bits(g[n])) for n in ("q", "k", "v"))
    seq = torch.from_numpy(g["seqused"]).cuda()
    out, lse = torch.ops.anima_flat.fa_fwd_k(q, k, v, seq)
    y = pkg.cross_attention_trimmed(q, k, v, seq, torch.from_numpy(g["ln_pad"]).cuda())
    torch.cuda.synchronize()
    parity(out, torch.from_numpy(g["out"]), name="golden masked out")
    parity(lse, torch.from_numpy(g["lse"]), max_abs=2e-3, rel_l2=2e-4, name="golden masked lse")
    parity(y.view(out.shape), torch.from_numpy(g["corrected"]), name="golden trimmed+corrected")


def test_golden_attention_backward(pkg):
    g = _g("attn_bwd_small.npz")
    q, k, v = (_dev(_bits(g[n])).requires_grad_(True) for n in ("q", "k", "v"))
    do = _dev(_bits(g["dout"]))
    out = pkg.attention(q, k, v)
    out.backward(do.reshape(out.shape))
    torch.cuda.synchronize()
    parity(q.grad, torch.from_numpy(g["dq"]), name="golden dq")
    parity(k.grad, torch.from_numpy(g["dk"]), name="golden dk")
    parity(v.grad, torch.from_numpy(g["dv"]), name="golden dv")


def test_golden_prologue(pkg):
    g = _g("prologue_small.npz")
    H, eps = int(g["heads"]), float(g["eps"])
    qkv = _dev(_bits(g["qkv"])).requires_grad_(True)
    qw = torch.from_numpy(g["q_weight"]).cuda().requires_grad_(True)
    kw = torch.from_numpy(g["k_weight"]).cuda().requires_grad_(True)
    cos, sin = torch.from_numpy(g["cos"]).cuda(), torch.from_numpy(g["sin"]).cuda()
    q, k, v = pkg.qkv_norm_rope(qkv, qw, kw, cos, sin, H, eps)
    dq, dk, dv = (_dev(_bits(g[n])) for n in ("dq", "dk", "dv"))
    torch.autograd.backward((q, k, v), (dq, dk, dv))
    torch.cuda.synchronize()
    parity(q, torch.from_numpy(g["q"]), name="golden q")
    parity(k, torch.from_numpy(g["k"]), name="golden k")
    parity(qkv.grad, torch.from_numpy(g["dqkv"]), name="golden dqkv")
    parity(qw.grad, torch.from_numpy(g["dq_weight"]), max_abs=2e-2 * max(1.0, float(np.abs(g["dq_weight"]).max())),
           name="golden dq_weight")
    parity(kw.grad, torch.from_numpy(g["dk_weight"]), max_abs=2e-2 * max(1.0, float(np.abs(g["dk_weight"]).max())),
           name="golden dk_weight")
    x = _dev(_bits(g["qkv"])).view(1, 12, 3, H * 128)[:, :, 0].contiguous().requires_grad_(True)
    w = torch.from_numpy(g["q_weight"]).cuda().requires_grad_(True)
    y = pkg.head_norm(x, w, H, eps)
    y.backward(dq)
    torch.cuda.synchronize()
    parity(y, torch.from_numpy(g["head_norm"]), name="golden head_norm")
    parity(x.grad.view(1, 12, H, 128), torch.from_numpy(g["head_norm_dx"]), name="golden head_norm dx")


def test_golden_ctx_scale(pkg):
    g = _g("ctx_scale_small.npz")
    out = _dev(_bits(g["out"])).requires_grad_(True)
    lse = torch.from_numpy(g["lse"]).cuda().requires_grad_(True)
    y = pkg.ctx_scale(out, lse, torch.from_numpy(g["ln_pad"]).cuda())
    y.backward(_dev(_bits(g["dy"])))
    torch.cuda.synchronize()
    parity(y, torch.from_numpy(g["y"]), name="golden ctx_scale y")
    parity(out.grad, torch.from_numpy(g["dout"]), name="golden ctx_scale dout")
    parity(lse.grad, torch.from_numpy(g["dlse"]), max_abs=2e-2 * max(1.0, float(np.abs(g["dlse"]).max())),
           name="golden ctx_scale dlse")
