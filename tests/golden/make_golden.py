"""Writes the golden fixtures under tests/golden/ (run: python tests/golden/make_golden.py).

The expected outputs are computed here in float64 NumPy from the closed-form
definitions of each function of the path, independently of the torch oracle
(oracle/attn_oracle.py) and of the HIP kernels, which the tests then check
against these vectors. Inputs are bf16 values, stored as their uint16 bit
patterns; outputs are stored as float32.

The reference repository holds no fixtures or golden vectors of its own for
this path, and its kernels (FlashAttention-4, Triton) cannot run here, so the
vectors come from the mathematics each reference function implements:
  attention       softmax(q k^T / sqrt(d)) v, LSE (src/attention.py:126-153)
  masked          keys >= seqused_k[b] excluded (src/attention.py:74-81)
  ctx_scale       out * 1/(1 + exp(ln_pad - lse)) (src/kernels/ctx_scale.py:19-35, 76-95)
  attention bwd   dV = P^T dO, dS = P (dP - rowsum(dP P)), dQ = s dS K, dK = s dS^T Q
  prologue        RMSNorm, bf16 round, rotate-half RoPE (src/kernels/rope.py:32-58, 244-274)
  rope tables     src/model.py:51-84
"""

from __future__ import annotations

from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent


# ------------------------------------------------------------ bf16 helpers --


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round float values to bf16 (round to nearest even) -> uint16 bit patterns."""
    u = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return rounded.astype(np.uint16)


def from_bits(b: np.ndarray) -> np.ndarray:
    return (b.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def round_bf16(x: np.ndarray) -> np.ndarray:
    return from_bits(bf16_bits(x))


def bf16_normal(rng: np.random.Generator, shape) -> tuple[np.ndarray, np.ndarray]:
    bits = bf16_bits(rng.standard_normal(shape))
    return bits, from_bits(bits)


# -------------------------------------------------------------- attention --


def attention(q, k, v, seqused=None):
    """q [B,Sq,H,d], k/v [B,Sk,H,d] float64 -> out [B,Sq,H,d], lse [B,H,Sq]."""
    d = q.shape[-1]
    s = np.einsum("bqhd,bkhd->bhqk", q, k) / np.sqrt(d)
    if seqused is not None:
        keys = np.arange(k.shape[1])
        mask = keys[None, :] < np.asarray(seqused)[:, None]
        s = np.where(mask[:, None, None, :], s, -np.inf)
    m = s.max(-1, keepdims=True)
    e = np.exp(s - m)
    den = e.sum(-1, keepdims=True)
    p = e / den
    lse = (m + np.log(den))[..., 0]
    return np.einsum("bhqk,bkhd->bqhd", p, v), lse, p


def attention_backward(q, k, v, dout):
    d = q.shape[-1]
    scale = 1.0 / np.sqrt(d)
    _, _, p = attention(q, k, v)
    dv = np.einsum("bhqk,bqhd->bkhd", p, dout)
    dp = np.einsum("bqhd,bkhd->bhqk", dout, v)
    ds = p * (dp - (dp * p).sum(-1, keepdims=True))
    dq = scale * np.einsum("bhqk,bkhd->bqhd", ds, k)
    dk = scale * np.einsum("bhqk,bqhd->bkhd", ds, q)
    return dq, dk, dv


def ctx_gain(lse, ln_pad):
    """[B,H,S] gain 1/(1 + exp(ln_pad[b] - lse))."""
    return 1.0 / (1.0 + np.exp(ln_pad[:, None, None] - lse))


# --------------------------------------------------------------- prologue --


def rope_tables(h, w, head_dim, rope_scale=(1.0, 1.0)):
    dh = head_dim // 6 * 2
    dt = head_dim - 2 * dh
    ntk = dh / (dh - 2)
    ar = np.arange(0, dh, 2, dtype=np.float64) / dh
    fh = 1.0 / ((10000.0 * rope_scale[0] ** ntk) ** ar)
    fw = 1.0 / ((10000.0 * rope_scale[1] ** ntk) ** ar)
    ah = np.broadcast_to((np.arange(h)[:, None] * fh[None, :])[:, None, :], (h, w, len(fh)))
    aw = np.broadcast_to((np.arange(w)[:, None] * fw[None, :])[None, :, :], (h, w, len(fw)))
    at = np.zeros((h, w, dt // 2))
    ang = np.concatenate([at, ah, aw], axis=-1).reshape(h * w, -1)
    return np.cos(ang), np.sin(ang)


def norm_rope(x, w, cos, sin, eps, rotate):
    """x [B,S,H,hd] float64 -> bf16-rounded output, the reference's order."""
    half = x.shape[-1] // 2
    rstd = 1.0 / np.sqrt((x * x).sum(-1, keepdims=True) / x.shape[-1] + eps)
    y = round_bf16(x * rstd * w)
    if not rotate:
        return y
    a, b = y[..., :half], y[..., half:]
    c, s = cos[None, :, None, :], sin[None, :, None, :]
    return round_bf16(np.concatenate([a * c - b * s, b * c + a * s], axis=-1))


def norm_rope_backward(x, dout, w, cos, sin, eps, rotate):
    """(dx, dw) of norm_rope with the rounding treated as the identity."""
    half = x.shape[-1] // 2
    if rotate:
        da, db = dout[..., :half], dout[..., half:]
        c, s = cos[None, :, None, :], sin[None, :, None, :]
        g = np.concatenate([da * c + db * s, db * c - da * s], axis=-1)
    else:
        g = dout
    rstd = 1.0 / np.sqrt((x * x).sum(-1, keepdims=True) / x.shape[-1] + eps)
    xh = x * rstd
    u = g * w
    dx = rstd * (u - xh * (u * xh).mean(-1, keepdims=True))
    dw = (g * xh).reshape(-1, x.shape[-1]).sum(0)
    return dx, dw


# ------------------------------------------------------------------- main --


def main() -> None:
    rng = np.random.default_rng(20261201)
    d = 128

    # Self-attention with partial tiles on both sides, and its LSE.
    qb, q = bf16_normal(rng, (1, 37, 2, d))
    kb, k = bf16_normal(rng, (1, 45, 2, d))
    vb, v = bf16_normal(rng, (1, 45, 2, d))
    out, lse, _ = attention(q, k, v)
    np.savez_compressed(HERE / "attn_small.npz", q=qb, k=kb, v=vb,
                        out=out.astype(np.float32), lse=lse.astype(np.float32))

    # Key-length mask, padding correction, and the zero-padded equivalent.
    S_full = 50
    seqused = np.array([17, 40], dtype=np.int32)
    qb, q = bf16_normal(rng, (2, 33, 1, d))
    kb, k = bf16_normal(rng, (2, 40, 1, d))
    vb, v = bf16_normal(rng, (2, 40, 1, d))
    out_m, lse_m, _ = attention(q, k, v, seqused)
    ln_pad = np.log((S_full - seqused).astype(np.float64))
    corrected = out_m * ctx_gain(lse_m, ln_pad).transpose(0, 2, 1)[..., None]
    kp = np.zeros((2, S_full, 1, d))
    vp = np.zeros((2, S_full, 1, d))
    for b, n in enumerate(seqused):
        kp[b, :n] = k[b, :n]
        vp[b, :n] = v[b, :n]
    out_padded, _, _ = attention(q, kp, vp)
    assert np.allclose(corrected, out_padded, atol=1e-12), "padding identity"
    np.savez_compressed(HERE / "masked_small.npz", q=qb, k=kb, v=vb, seqused=seqused,
                        s_full=np.int32(S_full), ln_pad=ln_pad.astype(np.float32),
                        out=out_m.astype(np.float32), lse=lse_m.astype(np.float32),
                        corrected=corrected.astype(np.float32))

    # Attention backward.
    qb, q = bf16_normal(rng, (1, 20, 1, d))
    kb, k = bf16_normal(rng, (1, 24, 1, d))
    vb, v = bf16_normal(rng, (1, 24, 1, d))
    db_, do = bf16_normal(rng, (1, 20, 1, d))
    dq, dk, dv = attention_backward(q, k, v, do)
    np.savez_compressed(HERE / "attn_bwd_small.npz", q=qb, k=kb, v=vb, dout=db_,
                        dq=dq.astype(np.float32), dk=dk.astype(np.float32),
                        dv=dv.astype(np.float32))

    # Prologue forward and backward (H=2, S=12 tokens of a 3 x 4 grid).
    H, S, eps = 2, 12, 1e-6
    cos, sin = rope_tables(3, 4, d, (4.0, 4.0))
    cos32, sin32 = cos.astype(np.float32), sin.astype(np.float32)
    qkvb, qkv = bf16_normal(rng, (1, S, 3 * H * d))
    qw = (1.0 + 0.02 * rng.standard_normal(d)).astype(np.float32)
    kw = (1.0 + 0.02 * rng.standard_normal(d)).astype(np.float32)
    x = qkv.reshape(1, S, 3, H, d)
    c64, s64 = cos32.astype(np.float64), sin32.astype(np.float64)
    qo = norm_rope(x[:, :, 0], qw.astype(np.float64), c64, s64, eps, True)
    ko = norm_rope(x[:, :, 1], kw.astype(np.float64), c64, s64, eps, True)
    dqb, dqo = bf16_normal(rng, (1, S, H, d))
    dkb, dko = bf16_normal(rng, (1, S, H, d))
    dvb, dvo = bf16_normal(rng, (1, S, H, d))
    dxq, dqw = norm_rope_backward(x[:, :, 0], dqo, qw.astype(np.float64), c64, s64, eps, True)
    dxk, dkw = norm_rope_backward(x[:, :, 1], dko, kw.astype(np.float64), c64, s64, eps, True)
    dqkv = np.stack([dxq, dxk, dvo], axis=2).reshape(1, S, 3 * H * d)
    hn = norm_rope(x[:, :, 0], qw.astype(np.float64), None, None, eps, False)
    dhn, dhw = norm_rope_backward(x[:, :, 0], dqo, qw.astype(np.float64), None, None, eps, False)
    np.savez_compressed(HERE / "prologue_small.npz", qkv=qkvb, q_weight=qw, k_weight=kw,
                        cos=cos32, sin=sin32, eps=np.float64(eps), heads=np.int32(H),
                        q=qo.astype(np.float32), k=ko.astype(np.float32),
                        dq=dqb, dk=dkb, dv=dvb, dqkv=dqkv.astype(np.float32),
                        dq_weight=dqw.astype(np.float32), dk_weight=dkw.astype(np.float32),
                        head_norm=hn.astype(np.float32), head_norm_dx=dhn.astype(np.float32),
                        head_norm_dw=dhw.astype(np.float32))

    # Rotary tables of a 5 x 7 grid, both frequency scales.
    c1, s1 = rope_tables(5, 7, d, (1.0, 1.0))
    c4, s4 = rope_tables(5, 7, d, (4.0, 4.0))
    np.savez_compressed(HERE / "rope_tables.npz", cos1=c1, sin1=s1, cos4=c4, sin4=s4)

    # ctx_scale forward and backward.
    ob, o = bf16_normal(rng, (2, 9, 3, d))
    lse_c = rng.standard_normal((2, 3, 9)) * 2 + 3
    lnp = np.array([-np.inf, 2.5])
    dyb, dy = bf16_normal(rng, (2, 9, 3, d))
    gain = ctx_gain(lse_c, lnp).transpose(0, 2, 1)[..., None]
    y = o * gain
    dlse = ((dy * o).sum(-1, keepdims=True) * gain * (1 - gain))[..., 0].transpose(0, 2, 1)
    np.savez_compressed(HERE / "ctx_scale_small.npz", out=ob, lse=lse_c.astype(np.float32),
                        ln_pad=lnp.astype(np.float32), dy=dyb, y=y.astype(np.float32),
                        dout=(dy * gain).astype(np.float32), dlse=dlse.astype(np.float32))
    print("wrote", sorted(p.name for p in HERE.glob("*.npz")))


if __name__ == "__main__":
    main()
