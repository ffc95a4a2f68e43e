"""CPU fp32 oracle of anima-flat's DiT attention path.

TEST INFRASTRUCTURE ONLY. This module restates the reference's arithmetic on
the CPU in float32 (float64 where a caller asks) so the HIP kernels can be
checked against it. Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import it, and only as the checker (or, in bench.py, as
the timed CPU baseline); no product code path calls it.

Every function names the reference lines (paths under anima-flat's src/) it
follows. The reference itself cannot run here (FlashAttention-4, Triton and an
NVIDIA GPU are required), so each function is pinned instead by the checks in
tests/test_oracle.py: float64 NumPy golden vectors written by
tests/golden/make_golden.py, closed forms and invariants, and gradcheck.

Storage rounding: the reference stores activations in bf16 between kernels.
`round_to=torch.bfloat16` reproduces that at the same points (after the
normalisation, rope.py:47-48, and on the stored outputs); `round_to=None`
keeps everything in the working dtype (used for gradcheck).
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F
from torch.nn.attention import SDPBackend, sdpa_kernel

BF16 = torch.bfloat16


def _round(x: torch.Tensor, round_to: torch.dtype | None) -> torch.Tensor:
    return x if round_to is None else x.to(round_to).to(x.dtype)


# ---------------------------------------------------------------- prologue --


def rms_norm_heads(
    x: torch.Tensor, weight: torch.Tensor, eps: float, round_to: torch.dtype | None = BF16
) -> torch.Tensor:
    """y = x * rsqrt(mean(x^2) + eps) * w over the last dim, then rounded.

    src/kernels/rope.py:41-48: rstd from the sum over both halves divided by
    head_dim, multiply by rstd then by the weight, round to the storage dtype.
    """
    rstd = torch.rsqrt(x.pow(2).sum(-1, keepdim=True) / x.shape[-1] + eps)
    return _round(x * rstd * weight, round_to)


def rotate_half(y: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """Rotate-half RoPE of y [B, S, H, hd] with cos/sin [S, hd/2].

    src/kernels/rope.py:49-53: pairs (a, b) = (y[i], y[i + hd/2]),
    out_a = a cos - b sin, out_b = b cos + a sin; position = token index in its
    sequence (rope.py:80).
    """
    half = y.shape[-1] // 2
    a, b = y[..., :half], y[..., half:]
    c = cos[None, :, None, :].to(y.dtype)
    s = sin[None, :, None, :].to(y.dtype)
    return torch.cat([a * c - b * s, b * c + a * s], dim=-1)


def qkv_norm_rope(
    qkv: torch.Tensor,
    q_weight: torch.Tensor,
    k_weight: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    heads: int,
    eps: float = 1e-5,
    round_to: torch.dtype | None = BF16,
    dtype: torch.dtype = torch.float32,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(q, k, v) [B, S, H, hd] from qkv [B, S, 3*H*hd].

    src/kernels/rope.py:61-143 and 616-645: q, k sections normalised with their
    weights and rotated; v passed through; q, k stored rounded.
    """
    B, S, _ = qkv.shape
    hd = 2 * cos.shape[1]
    x = qkv.to(dtype).reshape(B, S, 3, heads, hd)
    q = rms_norm_heads(x[:, :, 0], q_weight.to(dtype), eps, round_to)
    k = rms_norm_heads(x[:, :, 1], k_weight.to(dtype), eps, round_to)
    q = _round(rotate_half(q, cos.to(dtype), sin.to(dtype)), round_to)
    k = _round(rotate_half(k, cos.to(dtype), sin.to(dtype)), round_to)
    return q, k, x[:, :, 2]


def qkv_proj_norm_rope(
    hid: torch.Tensor,
    weight: torch.Tensor,
    q_weight: torch.Tensor,
    k_weight: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    heads: int,
    eps: float = 1e-5,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(q, k, v) of the block's QKV projection followed by the prologue
    (src/model.py:308-316): qkv = hid @ weight^T (nn.Linear without bias,
    model.py:134) accumulated in float32 and rounded to bf16, as the bf16 GEMM
    writes it, then `qkv_norm_rope`; v is the bf16 projection output."""
    qkv = (hid.float() @ weight.float().T).to(BF16)
    q, k, v = qkv_norm_rope(qkv, q_weight, k_weight, cos, sin, heads, eps)
    return q, k, v.to(BF16)


def head_norm(
    x: torch.Tensor,
    weight: torch.Tensor,
    heads: int,
    eps: float = 1e-5,
    round_to: torch.dtype | None = BF16,
    dtype: torch.dtype = torch.float32,
) -> torch.Tensor:
    """Per-head RMSNorm [B, S, H*hd] -> [B, S, H, hd] (src/kernels/rope.py:146-172)."""
    B, S, _ = x.shape
    hd = weight.numel()
    return rms_norm_heads(x.to(dtype).reshape(B, S, heads, hd), weight.to(dtype), eps, round_to)


def proj_head_norm(
    x: torch.Tensor, weight: torch.Tensor, norm_weight: torch.Tensor, heads: int, eps: float = 1e-5
) -> torch.Tensor:
    """q of the cross-attention, src/model.py:324: head_norm(b.xq(hid), ...) with
    b.xq an nn.Linear without bias (model.py:138); the projection accumulated in
    float32 and rounded to bf16 as the GEMM writes it, then `head_norm`."""
    y = (x.float() @ weight.float().T).to(BF16)
    return head_norm(y.float(), norm_weight, heads, eps)


def kv_proj_norm(
    ctx: torch.Tensor, weight: torch.Tensor, k_weight: torch.Tensor, heads: int, eps: float = 1e-5
) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-layer context keys and values, src/model.py:256-258:
    k, v = b.xkv(ctx).view(B, S, 2, H, hd).unbind(2) (b.xkv an nn.Linear without
    bias, model.py:139), k = F.rms_norm(k, (hd,), b.xk_norm.to(k.dtype), eps):
    the projection rounded to bf16, the norm in float32 with the weight rounded
    to bf16, the result rounded to bf16; v as projected."""
    B, S, _ = ctx.shape
    hd = k_weight.numel()
    kv = (ctx.float() @ weight.float().T).to(BF16).float().view(B, S, 2, heads, hd)
    k = rms_norm_heads(kv[:, :, 0], k_weight.to(BF16).float(), eps)
    return k, kv[:, :, 1]


def qkv_norm_rope_backward(
    qkv: torch.Tensor,
    dq: torch.Tensor,
    dk: torch.Tensor,
    dv: torch.Tensor,
    q_weight: torch.Tensor,
    k_weight: torch.Tensor,
    cos: torch.Tensor,
    sin: torch.Tensor,
    heads: int,
    eps: float = 1e-5,
    dtype: torch.dtype = torch.float32,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(dqkv, dq_weight, dk_weight) by autograd through `qkv_norm_rope`.

    The storage rounding is differentiated as the identity, as the reference's
    hand-written backward does (src/kernels/rope.py:244-274: inverse rotation,
    then rstd * (u - xhat * mean(u * xhat)), weight grads sum(dy' * xhat)).
    """
    x = qkv.to(dtype).detach().requires_grad_(True)
    qw = q_weight.to(dtype).detach().requires_grad_(True)
    kw = k_weight.to(dtype).detach().requires_grad_(True)
    q, k, v = qkv_norm_rope(x, qw, kw, cos, sin, heads, eps, round_to=None, dtype=dtype)
    torch.autograd.backward((q, k, v), (dq.to(dtype), dk.to(dtype), dv.to(dtype)))
    return x.grad, qw.grad, kw.grad


def head_norm_backward(
    x: torch.Tensor,
    dy: torch.Tensor,
    weight: torch.Tensor,
    heads: int,
    eps: float = 1e-5,
    dtype: torch.dtype = torch.float32,
) -> tuple[torch.Tensor, torch.Tensor]:
    """(dx, dweight) by autograd through `head_norm` (src/kernels/rope.py:386-471)."""
    xx = x.to(dtype).detach().requires_grad_(True)
    w = weight.to(dtype).detach().requires_grad_(True)
    y = head_norm(xx, w, heads, eps, round_to=None, dtype=dtype)
    y.backward(dy.to(dtype).reshape(y.shape))
    return xx.grad, w.grad


# --------------------------------------------------------------- attention --


def attention_sdpa(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor:
    """softmax(q k^T / sqrt(hd)) v on [B, S, H, hd] via torch SDPA, math backend.

    The reference's non-FA4 path (src/attention.py:150-153). Returns
    [B, Sq, H, hd] in q's dtype (call with float32 tensors).
    """
    with sdpa_kernel(SDPBackend.MATH):
        out = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2))
    return out.transpose(1, 2)


def attention_lse(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    seqused_k: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """(out [B,Sq,H,hd], lse [B,H,Sq]) with an optional key-length mask.

    Keys j >= seqused_k[b] are excluded (FA4's seqused_k, src/attention.py:74-81);
    lse is the natural-log log-sum-exp of the scaled scores over the attended
    keys (the LSE FA4 returns, checked at src/attention.py:48-52).
    """
    scale = 1.0 / math.sqrt(q.shape[-1])
    s = torch.einsum("bqhd,bkhd->bhqk", q, k) * scale
    if seqused_k is not None:
        keys = torch.arange(k.shape[1], device=q.device)
        keep = keys[None, :] < seqused_k.to(q.device)[:, None].long()
        s = s.masked_fill(~keep[:, None, None, :], float("-inf"))
    lse = torch.logsumexp(s, dim=-1)
    p = torch.exp(s - lse[..., None])
    out = torch.einsum("bhqk,bkhd->bqhd", p, v)
    return out, lse


def ctx_scale(out: torch.Tensor, lse: torch.Tensor, ln_pad: torch.Tensor) -> torch.Tensor:
    """out * 1/(1 + exp(ln_pad[b] - lse[b,h,s])) (src/kernels/ctx_scale.py:19-35)."""
    gain = 1.0 / (1.0 + torch.exp(ln_pad[:, None, None] - lse))  # [B, H, S]
    return out * gain.transpose(1, 2)[..., None]


def ctx_scale_backward(
    out: torch.Tensor, lse: torch.Tensor, ln_pad: torch.Tensor, dy: torch.Tensor
) -> tuple[torch.Tensor, torch.Tensor]:
    """(dout, dlse) of `ctx_scale` (src/kernels/ctx_scale.py:76-95):
    dout = dy g, dlse = sum_d(dy out) g (1 - g)."""
    gain = (1.0 / (1.0 + torch.exp(ln_pad[:, None, None] - lse))).transpose(1, 2)[..., None]
    dout = dy * gain
    dlse = ((dy * out).sum(-1, keepdim=True) * gain * (1.0 - gain))[..., 0].transpose(1, 2)
    return dout, dlse


def context_lengths(ctx: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """Key lengths and log padding of a zero-padded text context (src/model.py:248-253).

    length[b] = 1-based index of the last row of ctx[b] with any element != 0
    (at least 1), seqused = length as int32, ln_pad = log(S - length) in
    float32 (-inf when nothing is padded). -0.0 compares equal to 0; NaN does
    not.
    """
    S = ctx.shape[1]
    index = torch.arange(1, S + 1)
    lengths = ((ctx != 0).any(-1) * index).amax(1).clamp_min(1)
    return lengths.to(torch.int32), torch.log((S - lengths).float())


def gelu_as(x: torch.Tensor) -> torch.Tensor:
    """GELU with the Abramowitz-Stegun 7.1.26 erf approximation (src/kernels/fp8.py:260-270)."""
    z = x * 0.7071067811865476
    az = z.abs()
    t = 1.0 / (1.0 + 0.3275911 * az)
    poly = ((((1.061405429 * t - 1.453152027) * t + 1.421413741) * t - 0.284496736) * t + 0.254829592) * t
    y = 1.0 - poly * torch.exp(-az * az)
    return 0.5 * x * (1.0 + torch.where(z < 0, -y, y))


def rowquant(x: torch.Tensor, gelu: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-row FP8 quantisation (src/kernels/fp8.py:275-292, op :295-310).

    y = x (or GELU(x)) in float32, scale = max(max|y|, 1e-12) / 448 per row,
    q = float8_e4m3fn(clamp(y / scale, -448, 448)) (round to nearest even).
    Returns (q [B, S, K], scale [B*S, 1] float32).
    """
    B, S, K = x.shape
    y = x.float()
    if gelu:
        y = gelu_as(y)
    scale = y.abs().amax(-1, keepdim=True).clamp_min(1e-12) / 448.0
    q = (y / scale).clamp(-448.0, 448.0).to(torch.float8_e4m3fn)
    return q, scale.reshape(B * S, 1)


def cross_attention_trimmed(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    seqused_k: torch.Tensor,
    ln_pad: torch.Tensor,
) -> torch.Tensor:
    """Masked attention followed by the padding correction (src/attention.py:156-180)."""
    out, lse = attention_lse(q, k, v, seqused_k)
    return ctx_scale(out, lse, ln_pad)


def attention_backward(
    q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, dout: torch.Tensor
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(dq, dk, dv) by autograd through `attention_sdpa` (what FA4's backward,
    src/attention.py:91-103, computes)."""
    qq, kk, vv = (t.detach().requires_grad_(True) for t in (q, k, v))
    out = attention_sdpa(qq, kk, vv)
    out.backward(dout)
    return qq.grad, kk.grad, vv.grad


def attention_backward_rows(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    dout: torch.Tensor,
    qrows: torch.Tensor,
    krows: torch.Tensor,
    chunk: int = 1024,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(dq[:, qrows], dk[:, krows], dv[:, krows]) of `attention_sdpa` for long
    sequences, from the closed-form softmax gradient (what FA4's backward,
    src/attention.py:91-103, computes), without the full [Sq, Sk] matrix:

        P = softmax(s), s = q k^T / sqrt(hd), D_i = dO_i . O_i,
        dS_ij = P_ij (dO_i . v_j - D_i),
        dq_i = sum_j dS_ij k_j / sqrt(hd), dk_j = sum_i dS_ij q_i / sqrt(hd),
        dv_j = sum_i P_ij dO_i.

    Query rows are processed `chunk` at a time. Float32 throughout.
    """
    q, k, v, dout = (t.float() for t in (q, k, v, dout))
    scale = 1.0 / math.sqrt(q.shape[-1])
    kr, vr = k[:, krows], v[:, krows]
    dk = torch.zeros_like(kr)
    dv = torch.zeros_like(vr)
    qsel = torch.zeros(q.shape[1], dtype=torch.bool)
    qsel[qrows] = True
    dq = torch.zeros_like(q[:, qrows])
    done = 0
    for c0 in range(0, q.shape[1], chunk):
        qc, doc = q[:, c0 : c0 + chunk], dout[:, c0 : c0 + chunk]
        s = torch.einsum("bqhd,bkhd->bhqk", qc, k) * scale
        p = torch.softmax(s, dim=-1)
        oc = torch.einsum("bhqk,bkhd->bqhd", p, v)
        dD = (doc * oc).sum(-1).transpose(1, 2)  # [B, H, c]
        # key rows of the sample: their columns of P and dS
        pk = p[..., krows]
        dsk = pk * (torch.einsum("bqhd,bkhd->bhqk", doc, vr) - dD[..., None])
        dv += torch.einsum("bhqk,bqhd->bkhd", pk, doc)
        dk += torch.einsum("bhqk,bqhd->bkhd", dsk, qc) * scale
        # query rows of the sample inside this chunk
        sel = qsel[c0 : c0 + chunk].nonzero()[:, 0]
        if sel.numel():
            ps = p[:, :, sel]
            dss = ps * (torch.einsum("bqhd,bkhd->bhqk", doc[:, sel], v) - dD[:, :, sel, None])
            dq[:, done : done + sel.numel()] = torch.einsum("bhqk,bkhd->bqhd", dss, k) * scale
            done += sel.numel()
    return dq, dk, dv


# ------------------------------------------------------------ rope tables --


def rope_tables(
    h: int, w: int, head_dim: int, rope_scale: tuple = (1.0, 1.0)
) -> tuple[torch.Tensor, torch.Tensor]:
    """cos/sin [h*w, head_dim/2] float32 (src/model.py:51-84).

    Slot layout for head_dim 128: 22 time slots (angle 0, T = 1), then 21
    height slots (angle = row * f_i), then 21 width slots (angle = col * f_i),
    f_i = 1 / (10000 * scale^(dh/(dh-2)))^(2i/dh), dh = head_dim // 6 * 2.
    """
    dh = head_dim // 6 * 2
    dt = head_dim - 2 * dh
    ntk = dh / (dh - 2)
    ar = torch.arange(0, dh, 2, dtype=torch.float32) / dh
    fh = 1.0 / ((10000.0 * rope_scale[0] ** ntk) ** ar)
    fw = 1.0 / ((10000.0 * rope_scale[1] ** ntk) ** ar)
    yy = torch.arange(h, dtype=torch.float32)
    xx = torch.arange(w, dtype=torch.float32)
    ah = (yy[:, None] * fh[None, :])[:, None, :].expand(h, w, -1)
    aw = (xx[:, None] * fw[None, :])[None, :, :].expand(h, w, -1)
    at = torch.zeros(h, w, dt // 2)
    ang = torch.cat([at, ah, aw], dim=-1).reshape(h * w, -1)
    return ang.cos(), ang.sin()


# ------------------------------------------------------------------ inputs --

# Grid (h, w) of the image-token configurations (patch 2 over the latent).
GRIDS = {1024: (32, 32), 4096: (64, 64), 9216: (96, 96)}


def bf16_normal(shape, generator: torch.Generator) -> torch.Tensor:
    """N(0,1) drawn in fp32 on the CPU and rounded through bf16 (returned fp32)."""
    return torch.randn(shape, generator=generator).to(BF16).float()


def norm_weight(hd: int, generator: torch.Generator) -> torch.Tensor:
    """RMSNorm weight 1 + 0.02 N(0,1), float32."""
    return 1.0 + 0.02 * torch.randn(hd, generator=generator)


def prologue_inputs(
    B: int, S: int, H: int = 16, hd: int = 128, seed: int = 1000, rope_scale=(1.0, 1.0)
) -> dict[str, torch.Tensor]:
    """qkv [B,S,3*H*hd] ~ N(0,1) (bf16 values), q/k weights, cos/sin for the
    image grid of S tokens (a 1 x S strip when S is not a listed grid)."""
    g = torch.Generator().manual_seed(seed)
    qkv = bf16_normal((B, S, 3 * H * hd), g)
    qw = norm_weight(hd, g)
    kw = norm_weight(hd, g)
    gh, gw = GRIDS.get(S, (1, S))
    cos, sin = rope_tables(gh, gw, hd, rope_scale)
    return {"qkv": qkv, "q_weight": qw, "k_weight": kw, "cos": cos, "sin": sin}
