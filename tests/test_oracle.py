"""Pins the CPU oracle (oracle/attn_oracle.py) before it is trusted as the checker.

Three kinds of evidence, none of which re-types the oracle's own formulas:
  * golden vectors written by tests/golden/make_golden.py in float64 NumPy;
  * closed forms and invariants (permutation invariance, constant V, one key,
    logsumexp, the padding identity, rotation norms, relative positions);
  * torch.autograd.gradcheck in float64 for every backward.
The "planted mistake" tests perturb the oracle (a flipped rotation sign, a
dropped eps, a transposed table) and show that the checks above catch it.
"""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attn_oracle as ref

GOLD = Path(__file__).resolve().parent / "golden"


def _bits(a: np.ndarray) -> torch.Tensor:
    """uint16 bf16 bit patterns -> float32 tensor."""
    return torch.from_numpy((a.astype(np.uint32) << 16).view(np.float32).copy())


def _load(name):
    return np.load(GOLD / name, allow_pickle=False)


def _close(a, e, atol, rtol=0.0):
    a = torch.as_tensor(a, dtype=torch.float64)
    e = torch.as_tensor(np.asarray(e), dtype=torch.float64)
    assert a.shape == e.shape
    err = (a - e).abs().max().item()
    assert torch.allclose(a, e, atol=atol, rtol=rtol), f"max err {err:.3e}"


# ---------------------------------------------------------------- golden --


def test_attention_matches_golden():
    g = _load("attn_small.npz")
    q, k, v = _bits(g["q"]), _bits(g["k"]), _bits(g["v"])
    _close(ref.attention_sdpa(q, k, v), g["out"], atol=2e-6)
    out, lse = ref.attention_lse(q, k, v)
    _close(out, g["out"], atol=2e-6)
    _close(lse, g["lse"], atol=2e-6)


def test_masked_attention_and_padding_correction_match_golden():
    g = _load("masked_small.npz")
    q, k, v = _bits(g["q"]), _bits(g["k"]), _bits(g["v"])
    seq = torch.from_numpy(g["seqused"])
    out, lse = ref.attention_lse(q, k, v, seq)
    _close(out, g["out"], atol=2e-6)
    _close(lse, g["lse"], atol=2e-6)
    y = ref.cross_attention_trimmed(q, k, v, seq, torch.from_numpy(g["ln_pad"]))
    _close(y, g["corrected"], atol=2e-6)


def test_attention_backward_matches_golden():
    g = _load("attn_bwd_small.npz")
    q, k, v, do = (_bits(g[n]) for n in ("q", "k", "v", "dout"))
    dq, dk, dv = ref.attention_backward(q, k, v, do)
    _close(dq, g["dq"], atol=2e-5)
    _close(dk, g["dk"], atol=2e-5)
    _close(dv, g["dv"], atol=2e-5)


def test_prologue_matches_golden():
    g = _load("prologue_small.npz")
    qkv = _bits(g["qkv"])
    qw, kw = torch.from_numpy(g["q_weight"]), torch.from_numpy(g["k_weight"])
    cos, sin = torch.from_numpy(g["cos"]), torch.from_numpy(g["sin"])
    H, eps = int(g["heads"]), float(g["eps"])
    q, k, v = ref.qkv_norm_rope(qkv, qw, kw, cos, sin, H, eps)
    # float32 vs float64 intermediates can flip a bf16 rounding: one ulp, rarely.
    for got, exp in ((q, g["q"]), (k, g["k"])):
        diff = (got.double() - torch.from_numpy(exp).double()).abs()
        assert (diff > 0).double().mean().item() < 0.01
        assert diff.max().item() <= 2 ** -7 * max(1.0, float(np.abs(exp).max()))
    assert torch.equal(v, qkv.view(1, 12, 3, H, 128)[:, :, 2])
    hn = ref.head_norm(qkv.view(1, 12, 3, H * 128)[:, :, 0], qw, H, eps)
    diff = (hn.double() - torch.from_numpy(g["head_norm"]).double()).abs()
    assert (diff > 0).double().mean().item() < 0.01


def test_prologue_backward_matches_golden():
    g = _load("prologue_small.npz")
    qkv = _bits(g["qkv"])
    qw, kw = torch.from_numpy(g["q_weight"]), torch.from_numpy(g["k_weight"])
    cos, sin = torch.from_numpy(g["cos"]), torch.from_numpy(g["sin"])
    H, eps = int(g["heads"]), float(g["eps"])
    dq, dk, dv = (_bits(g[n]) for n in ("dq", "dk", "dv"))
    dqkv, dqw, dkw = ref.qkv_norm_rope_backward(qkv, dq, dk, dv, qw, kw, cos, sin, H, eps)
    _close(dqkv, g["dqkv"], atol=1e-5)
    _close(dqw, g["dq_weight"], atol=1e-4)
    _close(dkw, g["dk_weight"], atol=1e-4)
    x = qkv.view(1, 12, 3, H * 128)[:, :, 0].contiguous()
    dx, dw = ref.head_norm_backward(x, dq, qw, H, eps)
    _close(dx.view(1, 12, H, 128), g["head_norm_dx"], atol=1e-5)
    _close(dw, g["head_norm_dw"], atol=1e-4)


@pytest.mark.parametrize("scale,key", [((1.0, 1.0), "1"), ((4.0, 4.0), "4")])
def test_rope_tables_match_golden(scale, key):
    g = _load("rope_tables.npz")
    cos, sin = ref.rope_tables(5, 7, 128, scale)
    _close(cos, g["cos" + key], atol=3e-6)
    _close(sin, g["sin" + key], atol=3e-6)


def test_ctx_scale_matches_golden():
    g = _load("ctx_scale_small.npz")
    out, dy = _bits(g["out"]), _bits(g["dy"])
    lse, ln_pad = torch.from_numpy(g["lse"]), torch.from_numpy(g["ln_pad"])
    _close(ref.ctx_scale(out, lse, ln_pad), g["y"], atol=1e-6)
    dout, dlse = ref.ctx_scale_backward(out, lse, ln_pad, dy)
    _close(dout, g["dout"], atol=1e-6)
    _close(dlse, g["dlse"], atol=1e-5)


# ------------------------------------------------- closed forms, invariants --


def _rand(*shape, seed=0, dtype=torch.float64):
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed), dtype=dtype)


def test_attention_brute_force_small():
    q, k, v = _rand(2, 5, 3, 8, seed=1), _rand(2, 7, 3, 8, seed=2), _rand(2, 7, 3, 8, seed=3)
    out = ref.attention_sdpa(q, k, v)
    for b in range(2):
        for h in range(3):
            for i in range(5):
                s = [sum(q[b, i, h, t] * k[b, j, h, t] for t in range(8)) / math.sqrt(8) for j in range(7)]
                m = max(s)
                w = [math.exp(x - m) for x in s]
                z = sum(w)
                for t in range(8):
                    e = sum(w[j] * v[b, j, h, t] for j in range(7)) / z
                    assert abs(out[b, i, h, t].item() - e) < 1e-12


def test_attention_invariants():
    q, k, v = _rand(1, 9, 2, 16, seed=4), _rand(1, 11, 2, 16, seed=5), _rand(1, 11, 2, 16, seed=6)
    out = ref.attention_sdpa(q, k, v)
    perm = torch.randperm(11, generator=torch.Generator().manual_seed(7))
    torch.testing.assert_close(ref.attention_sdpa(q, k[:, perm], v[:, perm]), out)
    const = torch.ones_like(v) * 3.25
    torch.testing.assert_close(ref.attention_sdpa(q, k, const), torch.full_like(out, 3.25))
    one = ref.attention_sdpa(q, k[:, :1], v[:, :1])
    torch.testing.assert_close(one, v[:, :1].expand_as(one))
    _, lse = ref.attention_lse(q, k, v)
    s = torch.einsum("bqhd,bkhd->bhqk", q, k) / 4.0
    torch.testing.assert_close(lse, torch.from_numpy(np.log(np.exp(s.numpy()).sum(-1))))


def test_masked_equals_truncated_and_padding_identity():
    q, k, v = _rand(2, 6, 2, 8, seed=8), _rand(2, 10, 2, 8, seed=9), _rand(2, 10, 2, 8, seed=10)
    lens = torch.tensor([3, 10], dtype=torch.int32)
    out, _ = ref.attention_lse(q, k, v, lens)
    for b, n in enumerate(lens.tolist()):
        torch.testing.assert_close(out[b : b + 1], ref.attention_sdpa(q[b : b + 1], k[b : b + 1, :n], v[b : b + 1, :n]))
    S_full = 16
    kp, vp = torch.zeros(2, S_full, 2, 8, dtype=torch.float64), torch.zeros(2, S_full, 2, 8, dtype=torch.float64)
    for b, n in enumerate(lens.tolist()):
        kp[b, :n], vp[b, :n] = k[b, :n], v[b, :n]
    y = ref.cross_attention_trimmed(q, k, v, lens, torch.log((S_full - lens).double()))
    torch.testing.assert_close(y, ref.attention_sdpa(q, kp, vp))


def test_rms_norm_equals_functional_and_unit_rms():
    x = _rand(3, 4, 2, 128, seed=11, dtype=torch.float32)
    w = 1 + 0.02 * _rand(128, seed=12, dtype=torch.float32)
    y = ref.rms_norm_heads(x, w, 1e-6, round_to=None)
    torch.testing.assert_close(y, F.rms_norm(x, (128,), w, 1e-6))
    y1 = ref.rms_norm_heads(x, torch.ones(128), 1e-6, round_to=None)
    torch.testing.assert_close(y1.pow(2).mean(-1), torch.ones(3, 4, 2), atol=1e-4, rtol=0)


def test_rotation_norms_identity_and_relative_position():
    y = _rand(1, 6, 2, 128, seed=13)
    ang = _rand(6, 64, seed=14)
    r = ref.rotate_half(y, ang.cos(), ang.sin())
    pair = lambda t: t[..., :64] ** 2 + t[..., 64:] ** 2  # noqa: E731
    torch.testing.assert_close(pair(r), pair(y))
    torch.testing.assert_close(ref.rotate_half(y, torch.ones(6, 64, dtype=torch.float64), torch.zeros(6, 64, dtype=torch.float64)), y)
    # 1-D rotary: angle = position * f_i makes q_m . k_n depend on m - n only.
    f = 1.0 / (10000 ** (torch.arange(64, dtype=torch.float64) / 64))
    pos = torch.arange(6, dtype=torch.float64)
    a = pos[:, None] * f[None]
    q1 = _rand(1, 1, 1, 128, seed=15).expand(1, 6, 1, 128)
    k1 = _rand(1, 1, 1, 128, seed=16).expand(1, 6, 1, 128)
    qr, kr = ref.rotate_half(q1, a.cos(), a.sin()), ref.rotate_half(k1, a.cos(), a.sin())
    dots = (qr[0, :, None, 0] * kr[0, None, :, 0]).sum(-1)
    for shift in range(1, 4):
        diag = torch.diagonal(dots, offset=shift)
        torch.testing.assert_close(diag, diag[:1].expand_as(diag))


def test_qkv_projection_orientation_closed_form():
    """The fused-projection oracle with W = [P; I; 2I] (P a permutation, not
    symmetric): the q section is hid permuted by P's rows (a transposed weight
    would apply the inverse permutation), k is hid itself, v is exactly 2 hid."""
    g = torch.Generator().manual_seed(5)
    B, S, H = 2, 6, 2
    D = H * 128
    hid = ref.bf16_normal((B, S, D), g)
    perm = torch.randperm(D, generator=g)
    assert not torch.equal(perm, torch.argsort(perm))
    P = torch.zeros(D, D)
    P[torch.arange(D), perm] = 1.0
    w = torch.cat([P, torch.eye(D), 2 * torch.eye(D)]).to(torch.bfloat16)
    qw, kw = ref.norm_weight(128, g), ref.norm_weight(128, g)
    cos, sin = ref.rope_tables(2, 3, 128)
    q, k, v = ref.qkv_proj_norm_rope(hid, w, qw, kw, cos, sin, H, 1e-6)
    qkv = torch.cat([hid[..., perm], hid, 2 * hid], dim=-1)
    eq, ek, _ = ref.qkv_norm_rope(qkv, qw, kw, cos, sin, H, 1e-6)
    assert torch.equal(q, eq) and torch.equal(k, ek)
    assert torch.equal(v.float(), (2 * hid.float()).reshape(B, S, H, 128))
    wrong = torch.cat([hid[..., torch.argsort(perm)], hid, 2 * hid], dim=-1)
    assert not torch.equal(q, ref.qkv_norm_rope(wrong, qw, kw, cos, sin, H, 1e-6)[0])


def test_rope_table_structure():
    cos, sin = ref.rope_tables(4, 6, 128)
    assert cos.shape == (24, 64)
    assert torch.all(cos[:, :22] == 1) and torch.all(sin[:, :22] == 0)  # time slots: angle 0
    grid = cos.view(4, 6, 64)
    assert torch.all(grid[:, :, 22:43] == grid[:, :1, 22:43])  # height slots vary with the row only
    assert torch.all(grid[:, :, 43:] == grid[:1, :, 43:])  # width slots vary with the column only
    # slot 22 + i of row y: cos(y * 10000^(-2i/42)).
    i, y = 5, 3
    assert abs(grid[y, 0, 22 + i].item() - math.cos(y * 10000 ** (-2 * i / 42))) < 1e-6


# -------------------------------------------------------------- gradchecks --


def test_attention_backward_gradcheck():
    q, k, v = (_rand(1, 4, 2, 8, seed=s).requires_grad_(True) for s in (17, 18, 19))
    torch.autograd.gradcheck(lambda a, b, c: ref.attention_sdpa(a, b, c), (q, k, v))
    do = _rand(1, 4, 2, 8, seed=20)
    dq, dk, dv = ref.attention_backward(q.detach(), k.detach(), v.detach(), do)
    out = ref.attention_sdpa(q, k, v)
    gq, gk, gv = torch.autograd.grad(out, (q, k, v), do)
    torch.testing.assert_close((dq, dk, dv), (gq, gk, gv))


def test_chunked_sampled_backward_equals_autograd():
    """The closed-form, chunked backward on sampled rows (used at lengths where the
    full score matrix does not fit) against autograd, with chunks that split the
    sample unevenly and a last chunk that is partial."""
    g = torch.Generator().manual_seed(61)
    B, Sq, Sk, H = 2, 150, 97, 3
    q, do = (torch.randn(B, Sq, H, 16, generator=g, dtype=torch.float64) for _ in range(2))
    k, v = (torch.randn(B, Sk, H, 16, generator=g, dtype=torch.float64) for _ in range(2))
    dq, dk, dv = ref.attention_backward(q, k, v, do)
    qrows = torch.tensor([0, 3, 63, 64, 100, 149])
    krows = torch.tensor([0, 1, 50, 96])
    sq, sk, sv = ref.attention_backward_rows(q, k, v, do, qrows, krows, chunk=64)
    tol = dict(rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(sq, dq[:, qrows].float(), **tol)
    torch.testing.assert_close(sk, dk[:, krows].float(), **tol)
    torch.testing.assert_close(sv, dv[:, krows].float(), **tol)


def test_prologue_gradcheck():
    H, S = 1, 3
    cos, sin = ref.rope_tables(1, 3, 128)
    qkv = _rand(1, S, 3 * H * 128, seed=21).requires_grad_(True)
    qw = (1 + 0.1 * _rand(128, seed=22)).requires_grad_(True)
    kw = (1 + 0.1 * _rand(128, seed=23)).requires_grad_(True)
    fn = lambda x, a, b: ref.qkv_norm_rope(  # noqa: E731
        x, a, b, cos.double(), sin.double(), H, 1e-6, round_to=None, dtype=torch.float64)
    torch.autograd.gradcheck(fn, (qkv, qw, kw))
    x = _rand(1, S, H * 128, seed=24).requires_grad_(True)
    torch.autograd.gradcheck(lambda a, w: ref.head_norm(a, w, H, 1e-6, None, torch.float64), (x, qw))


def test_ctx_scale_gradcheck():
    out = _rand(1, 3, 2, 8, seed=25).requires_grad_(True)
    lse = _rand(1, 2, 3, seed=26).requires_grad_(True)
    ln_pad = torch.tensor([0.7], dtype=torch.float64)
    torch.autograd.gradcheck(lambda o, l: ref.ctx_scale(o, l, ln_pad), (out, lse))
    dy = _rand(1, 3, 2, 8, seed=27)
    dout, dlse = ref.ctx_scale_backward(out.detach(), lse.detach(), ln_pad, dy)
    go, gl = torch.autograd.grad(ref.ctx_scale(out, lse, ln_pad), (out, lse), dy)
    torch.testing.assert_close((dout, dlse), (go, gl))


# --------------------------------------------------------- planted mistakes --


def test_planted_rotation_sign_error_is_caught(monkeypatch):
    """A flipped sign in the rotation must fail the golden prologue check."""
    def wrong(y, cos, sin):
        half = y.shape[-1] // 2
        a, b = y[..., :half], y[..., half:]
        c, s = cos[None, :, None, :], sin[None, :, None, :]
        return torch.cat([a * c + b * s, b * c - a * s], dim=-1)

    monkeypatch.setattr(ref, "rotate_half", wrong)
    with pytest.raises(AssertionError):
        test_prologue_matches_golden()


def test_planted_missing_eps_and_wrong_scale_are_caught(monkeypatch):
    g = _load("attn_small.npz")
    q, k, v = _bits(g["q"]), _bits(g["k"]), _bits(g["v"])
    out, _ = ref.attention_lse(q * math.sqrt(2.0), k, v)  # scale 1/sqrt(64) instead of 1/sqrt(128)
    with pytest.raises(AssertionError):
        _close(out, g["out"], atol=2e-6)
    x = _rand(1, 2, 1, 128, seed=28, dtype=torch.float32) * 1e-4  # tiny rows: eps matters
    y_eps = ref.rms_norm_heads(x, torch.ones(128), 1e-2, round_to=None)
    y_no = ref.rms_norm_heads(x, torch.ones(128), 0.0, round_to=None)
    assert not torch.allclose(y_eps, y_no)


def test_planted_transposed_rope_table_is_caught():
    g = _load("rope_tables.npz")
    cos, _ = ref.rope_tables(7, 5, 128)  # h and w swapped
    with pytest.raises(AssertionError):
        _close(cos, g["cos1"], atol=3e-6)


def test_context_lengths_closed_form():
    """Hand-built paddings: the length is the last non-zero row, whatever lies before it."""
    ctx = torch.zeros(5, 40, 6)
    ctx[0, :7] = 1.0  # plain padding after 7 rows
    ctx[1, :30] = 1.0
    ctx[1, 10:20] = 0.0  # interior zeros do not end the sequence
    # ctx[2] all zero -> length 1
    ctx[3, :] = 2.0  # no padding -> ln_pad = -inf
    ctx[4, 12, 5] = -3.0  # a single non-zero element in row 12
    ctx[4, 20:25] = -0.0  # negative zeros count as zero
    seq, lnp = ref.context_lengths(ctx)
    assert seq.tolist() == [7, 30, 1, 40, 13] and seq.dtype == torch.int32
    expect = torch.tensor([math.log(33), math.log(10), math.log(39), -math.inf, math.log(27)])
    torch.testing.assert_close(lnp, expect.float())
    nan = torch.zeros(1, 9, 2)
    nan[0, 6, 1] = float("nan")  # NaN is not zero
    assert ref.context_lengths(nan)[0].tolist() == [7]


def test_rowquant_gelu_is_the_abramowitz_stegun_erf():
    """The GELU form is erf 7.1.26 (|error| <= 1.5e-7): against the exact erf GELU in float64."""
    x = torch.linspace(-8, 8, 20001, dtype=torch.float64)
    err = (ref.gelu_as(x) - F.gelu(x)).abs()
    assert (err <= 0.5 * x.abs() * 1.6e-7 + 1e-15).all()
    assert err.max() > 1e-9  # it is the approximation, not the exact function


def test_rowquant_known_answers_and_closed_form():
    # amax 448 -> scale 1: the codes are the e4m3fn round-to-nearest-even encodings.
    row = torch.tensor([[[448.0, 1.0625, 1.1875, 2.0**-10, 1.5 * 2.0**-9, -0.0, -3.0, 0.1]]])
    q, s = ref.rowquant(row)
    assert s.item() == 1.0
    # 1.0625 ties down to 1.0 (even), 1.1875 ties up to 1.25, 2^-10 ties to 0, 1.5*2^-9 to 2*2^-9
    assert q.view(torch.uint8).flatten()[:7].tolist() == [0x7E, 0x38, 0x3A, 0x00, 0x02, 0x80, 0xC4]
    g = torch.Generator().manual_seed(5)
    x = (torch.randn(3, 17, 64, generator=g) * torch.logspace(-6, 3, 64)).to(torch.bfloat16)
    x[1, 3] = 0.0  # an all-zero row
    q, s = ref.rowquant(x)
    xf = x.float().reshape(-1, 64)
    amax = xf.abs().amax(-1, keepdim=True)
    torch.testing.assert_close(s, amax.clamp_min(1e-12) / 448.0, rtol=0, atol=0)
    deq = q.float().reshape(-1, 64) * s
    # half an e4m3 ulp: 2^-4 relative for normals, 2^-10 * scale absolute below 2^-6 * scale
    bound = torch.maximum(xf.abs() * 2.0**-4, s * 2.0**-10)
    assert ((deq - xf).abs() <= bound * 1.0001).all()
    nz = amax.squeeze(-1) > 0
    assert (q.float().reshape(-1, 64).abs().amax(-1)[nz] == 448.0).all()
    assert (q.reshape(-1, 64)[~nz].float() == 0).all()
