"""GPU parity of the flash-attention kernels against the fp32 CPU oracle.

Tolerance (the north-star bar for bf16 forward and gradients): max-abs 2e-2
and relative L2 5e-3 against fp32 SDPA-math / autograd on the same bf16 input
values.
"""

from __future__ import annotations

import ctypes
import math
import sys

import pytest
import torch

from conftest import parity
from oracle import attn_oracle as ref

pytestmark = pytest.mark.gpu

BF = torch.bfloat16

# The kernel's LSE is the log of the sum of the bf16-rounded probabilities
# that weight V (so the output is exactly normalised); it differs from the
# fp32 logsumexp by ~2^-9 / sqrt(#keys) relative in the sum, i.e. < 1e-3 in lse.
LSE_TOL = dict(max_abs=2e-3, rel_l2=2e-4)
# A row whose softmax sits on one key carries that key's bf16-rounded p into the
# sum undiluted: up to 2^-8 relative (half an ulp just above a power of two),
# ln(1 + 2^-8) = 3.9e-3 in lse, unless m equals that key's score exactly.
LSE_TOL_PEAKED = dict(max_abs=4e-3, rel_l2=2e-4)


def _qkv(B, Sq, Sk, H, seed, hd=128):
    g = torch.Generator().manual_seed(seed)
    q = ref.bf16_normal((B, Sq, H, hd), g)
    k = ref.bf16_normal((B, Sk, H, hd), g)
    v = ref.bf16_normal((B, Sk, H, hd), g)
    return q, k, v


def _gpu(*ts, dev="cuda:0"):
    return [t.to(dev, BF) for t in ts]


@pytest.mark.parametrize(
    "B,Sq,Sk,H",
    [
        (1, 128, 128, 1),
        (1, 1024, 1024, 16),  # config 1 shape
        (2, 100, 77, 3),  # partial query block and partial key tile
        (1, 33, 1, 2),  # a single key
        (3, 1, 200, 2),  # a single query
        (2, 4096, 512, 4),  # cross-attention shape, untrimmed
    ],
)
def test_attention_forward(pkg, B, Sq, Sk, H):
    q, k, v = _qkv(B, Sq, Sk, H, seed=11 + Sq + Sk)
    out = pkg.attention(*_gpu(q, k, v))
    torch.cuda.synchronize()
    assert out.shape == (B, Sq, H * 128) and out.dtype == BF
    exp = ref.attention_sdpa(q, k, v).reshape(B, Sq, H * 128)
    parity(out, exp, name=f"fwd B{B} Sq{Sq} Sk{Sk} H{H}")


def test_attention_forward_lse(pkg):
    q, k, v = _qkv(2, 300, 260, 3, seed=5)
    out, lse = torch.ops.anima_flat.fa_fwd(*_gpu(q, k, v))
    torch.cuda.synchronize()
    eo, el = ref.attention_lse(q, k, v)
    assert lse.shape == (2, 3, 300) and lse.dtype == torch.float32
    parity(out, eo, name="fa_fwd out")
    parity(lse, el, **LSE_TOL, name="fa_fwd lse")


def test_attention_config2_full(pkg):
    """Config 2 at full size: B=1, 4096 tokens, 16 heads (q/k/v N(0,1))."""
    q, k, v = _qkv(1, 4096, 4096, 16, seed=1002)
    out = pkg.attention(*_gpu(q, k, v))
    torch.cuda.synchronize()
    exp = ref.attention_sdpa(q, k, v).reshape(1, 4096, 2048)
    parity(out, exp, name="config2 fwd")


def test_attention_strided_v_view(pkg, dev):
    """V as the strided view of qkv that qkv_norm_rope returns without grad."""
    B, S, H = 1, 192, 4
    g = torch.Generator().manual_seed(3)
    qkv = ref.bf16_normal((B, S, 3 * H * 128), g)
    x = qkv.view(B, S, 3, H, 128)
    q, k, v = x[:, :, 0], x[:, :, 1], x[:, :, 2]
    qkv_d = qkv.to(dev, BF)
    xd = qkv_d.view(B, S, 3, H, 128)
    out = pkg.attention(xd[:, :, 0], xd[:, :, 1], xd[:, :, 2])
    torch.cuda.synchronize()
    parity(out, ref.attention_sdpa(q, k, v).reshape(B, S, H * 128), name="strided views")


def test_attention_large_logits(pkg):
    """Scores far from zero exercise the lazy-rescale path (max grows across tiles)."""
    B, S, H = 1, 512, 2
    q, k, v = _qkv(B, S, S, H, seed=21)
    ramp = torch.linspace(0.2, 3.0, S)[None, :, None, None]
    k = (k * ramp).to(BF).float()  # later keys dominate
    q = (q * 2.0).to(BF).float()
    out = pkg.attention(*_gpu(q, k, v))
    torch.cuda.synchronize()
    parity(out, ref.attention_sdpa(q, k, v).reshape(B, S, H * 128), name="large logits")


def _spiked(B, Sq, Sk, H, delta, hot, seed):
    """N(0,1) q, k, v plus a shared unit direction u: every q row gets delta * u and
    the keys at positions `hot` become 20 u. A hot key's score then exceeds the
    other keys' (delta * N(0,1) along u) by ~17.6 delta, i.e. ~2.24 delta in log2
    units at scale 1/sqrt(128): past 64 from delta ~29, past 128 (p = inf with
    the first tile's max) from delta ~57."""
    q, k, v = _qkv(B, Sq, Sk, H, seed)
    g = torch.Generator().manual_seed(seed + 1)
    u = torch.randn(128, generator=g)
    u = u / u.norm()
    q = (q + delta * u).to(BF).float()
    k = k.clone()
    k[:, hot] = (20.0 * u).to(BF).float()
    return q, k, v


# Forward kernel forms: (AA_FWD_KERNEL, AA_FWD_FIRST_TILE_MAX); "1w" picks its
# form by the amount of work, "1w-ftm" forces the first-tile max with the fix-up
# launch, "1w-run" the running max.
FWD_FORMS = {"pp": ("pp", None), "1w": ("1w", None), "1w-ftm": ("1w", "1"), "1w-run": ("1w", "0")}


def _set_form(monkeypatch, form):
    kernel, ftm = FWD_FORMS[form]
    monkeypatch.setenv("AA_FWD_KERNEL", kernel)
    if ftm is None:
        monkeypatch.delenv("AA_FWD_FIRST_TILE_MAX", raising=False)
    else:
        monkeypatch.setenv("AA_FWD_FIRST_TILE_MAX", ftm)


def _clear_form(monkeypatch):
    monkeypatch.delenv("AA_FWD_KERNEL", raising=False)
    monkeypatch.delenv("AA_FWD_FIRST_TILE_MAX", raising=False)


@pytest.mark.parametrize("form", ["pp", "1w-ftm", "1w-run"])
@pytest.mark.parametrize("delta", [12.0, 33.0, 60.0])
@pytest.mark.parametrize(
    "B,Sq,Sk,H,lens,hot",
    [
        # 4 work items: split into 8 key ranges of 8 tiles; hot keys inside the
        # ranges of keys 2048-2559 and 3584-4095, past their first tiles.
        (1, 300, 4096, 2, None, [2118, 4091]),
        # 200 work items, no split (checked on sampled rows).
        (1, 2048, 2500, 25, None, [1000]),
        # key lengths: batch 1's key 2200 lies past its length (masked).
        (2, 300, 3000, 2, [3000, 1500], [900, 2200]),
    ],
)
def test_scores_far_above_the_first_tile(pkg, monkeypatch, form, delta, B, Sq, Sk, H, lens, hot):
    """Rows whose later scores exceed their first key tile's max by ~27, ~74 and
    ~134 in log2 units. The one-wave kernel's first-tile-max form keeps the first
    tile's max for the whole range: at ~27 its sums stay in range, at ~74 the row
    sums pass 2^64, at ~134 p overflows; the latter two write the rerun mark and
    the fix-up launch runs the item again with the running max. Every form is
    held to the oracle like any input; the LSE of these one-key rows to the bf16
    bound of LSE_TOL_PEAKED."""
    q, k, v = _spiked(B, Sq, Sk, H, delta, hot, seed=4400 + Sq + H)
    seq = torch.tensor(lens, dtype=torch.int32) if lens is not None else None
    _set_form(monkeypatch, form)
    qd, kd, vd = _gpu(q, k, v)
    if seq is None:
        out, lse = torch.ops.anima_flat.fa_fwd(qd, kd, vd)
    else:
        out, lse = torch.ops.anima_flat.fa_fwd_k(qd, kd, vd, seq.to("cuda"))
    torch.cuda.synchronize()
    _clear_form(monkeypatch)
    rows = torch.arange(Sq) if Sq <= 512 else torch.randperm(Sq, generator=torch.Generator().manual_seed(7))[:96]
    eo, el = ref.attention_lse(q[:, rows], k, v, seq)
    tag = f"{form} delta={delta} B{B} Sq{Sq} Sk{Sk} H{H} lens={lens}"
    parity(out[:, rows], eo, name=tag)
    parity(lse[:, :, rows], el, **LSE_TOL_PEAKED, name=f"lse {tag}")


def _random_long_cases(n, seed):
    """Seeded (B, Sq, Sk, H, lens, hot, delta): key ranges past 2048 (the one-wave
    kernel), ragged query and key counts, optional per-batch key lengths, and hot
    keys (scores ~2.24 delta log2 units above the rest) at random positions."""
    g = torch.Generator().manual_seed(seed)
    out = []
    for _ in range(n):
        B = int(torch.randint(1, 4, (1,), generator=g))
        H = int(torch.randint(1, 4, (1,), generator=g))
        Sq = int(torch.randint(1, 600, (1,), generator=g))
        Sk = int(torch.randint(2049, 4200, (1,), generator=g))
        lens = None
        if int(torch.randint(0, 2, (1,), generator=g)):
            lens = [int(torch.randint(1, Sk + 1, (1,), generator=g)) for _ in range(B)]
        hot = sorted({int(torch.randint(0, Sk, (1,), generator=g)) for _ in range(3)})
        delta = [0.0, 20.0, 40.0, 70.0][int(torch.randint(0, 4, (1,), generator=g))]
        out.append((B, Sq, Sk, H, lens, hot, delta))
    return out


@pytest.mark.parametrize("B,Sq,Sk,H,lens,hot,delta", _random_long_cases(10, seed=3003))
def test_random_first_tile_max_cases(pkg, monkeypatch, B, Sq, Sk, H, lens, hot, delta):
    """The first-tile-max form (forced) with its fix-up launch on seeded random shapes:
    key splits over partial last rounds, ragged tiles, key lengths that cut or skip the
    hot keys, and rows whose scores stay in range (delta 0, 20), pass 2^64 (40) or
    overflow (70). Out and LSE against the oracle."""
    q, k, v = _spiked(B, Sq, Sk, H, delta, hot, seed=5000 + Sq + Sk)
    seq = torch.tensor(lens, dtype=torch.int32) if lens is not None else None
    _set_form(monkeypatch, "1w-ftm")
    qd, kd, vd = _gpu(q, k, v)
    if seq is None:
        out, lse = torch.ops.anima_flat.fa_fwd(qd, kd, vd)
    else:
        out, lse = torch.ops.anima_flat.fa_fwd_k(qd, kd, vd, seq.to("cuda"))
    torch.cuda.synchronize()
    _clear_form(monkeypatch)
    eo, el = ref.attention_lse(q, k, v, seq)
    tag = f"B{B} Sq{Sq} Sk{Sk} H{H} lens={lens} hot={hot} delta={delta}"
    parity(out, eo, name=tag)
    parity(lse, el, **LSE_TOL_PEAKED, name=f"lse {tag}")


def test_stale_rerun_mark_in_output(pkg, dev, monkeypatch):
    """An output buffer that already holds the rerun mark everywhere (as a reused
    allocation might) is overwritten: the first-tile-max launch writes every element
    of a work item whose sums stayed in range, so the fix-up launch finds no mark."""
    _set_form(monkeypatch, "1w-ftm")
    A = sys.modules[pkg.__name__ + ".attention"]
    L = pkg._lib
    B, S, H = 1, 512, 2
    q, k, v = _qkv(B, S, 4096, H, seed=77)
    qd, kd, vd = _gpu(q, k, v)
    out = torch.full((B, S, H, 128), 0x7FC1, dtype=torch.int16, device=dev).view(BF)
    args = A._fwd_args(qd, kd, vd, out, None, None, None)
    ws = None
    need = L.lib().aa_attn_fwd_workspace(B, S, 4096, H, 128)
    if need:
        ws = torch.empty(need, dtype=torch.uint8, device=dev)
        args.workspace, args.workspace_bytes = ws.data_ptr(), need
    L.check(L.lib().aa_attn_fwd(ctypes.byref(args), L.stream(qd)), "attn_fwd")
    torch.cuda.synchronize()
    _clear_form(monkeypatch)
    parity(out, ref.attention_sdpa(q, k, v).reshape(B, S, H, 128), name="stale mark")


@pytest.mark.parametrize(
    "B,Sq,Sk,H,lens",
    [
        (2, 4096, 160, 16, None),  # 512 work items: two rounds on 256 CUs
        (1, 5120, 96, 15, None),  # 300 items: an uneven second round
        (4, 4096, 300, 16, [0, 1, 65, 300]),  # 1024 items; a batch without keys, one key, partial tiles
        (2, 1024, 300, 8, [0, 170]),  # 64 items split over key ranges; empty ranges
    ],
)
def test_large_grid_forward(pkg, B, Sq, Sk, H, lens):
    """More work items (256 queries of one (batch, head)) than CUs (several
    rounds of workgroups, an uneven last round), and a batch item with no keys."""
    q, k, v = _qkv(B, Sq, Sk, H, seed=71 + B)
    qd, kd, vd = _gpu(q, k, v)
    if lens is None:
        out, lse = torch.ops.anima_flat.fa_fwd(qd, kd, vd)
        seq = None
    else:
        seq = torch.tensor(lens, dtype=torch.int32)
        out, lse = torch.ops.anima_flat.fa_fwd_k(qd, kd, vd, seq.cuda())
    torch.cuda.synchronize()
    eo, el = ref.attention_lse(q, k, v, seq)
    keep = [b for b in range(B) if lens is None or lens[b] > 0]
    parity(out[keep], eo[keep], name=f"large grid out {B}x{Sq}x{Sk}x{H}")
    parity(lse[keep], el[keep], **LSE_TOL, name=f"large grid lse {B}x{Sq}x{Sk}x{H}")
    for b in range(B):
        if lens is not None and lens[b] == 0:  # no keys: O = 0, LSE = -inf
            assert torch.count_nonzero(out[b]).item() == 0
            assert torch.isneginf(lse[b]).all()


def test_forward_workspace(pkg):
    """A partial last round of work items is split over key ranges (bf16
    partial O and fp32 LSE in the workspace); a whole number of rounds needs none."""
    lib = pkg._lib.lib()
    if torch.cuda.get_device_properties(0).multi_processor_count != 256:
        pytest.skip("sizes below are for 256 CUs (MI355X)")
    assert lib.aa_attn_fwd_workspace(1, 4096, 4096, 16, 128) == 0  # config 2: one full round
    assert lib.aa_attn_fwd_workspace(2, 4096, 4096, 16, 128) == 0  # two full rounds
    # config 1: 64 items alone on 256 CUs -> 4 key ranges each, 256 x (128 bf16 + 1 fp32) per range
    assert lib.aa_attn_fwd_workspace(1, 1024, 1024, 16, 128) == 64 * 4 * 256 * (128 * 2 + 4)
    # config 4b: 576 items = 2 rounds + 64 -> the last 64 split 4 ways
    assert lib.aa_attn_fwd_workspace(1, 9216, 9216, 16, 128) == 64 * 4 * 256 * (128 * 2 + 4)


@pytest.mark.parametrize("lens", [[37, 80], [1, 64], [80, 80], [65, 3]])
def test_masked_forward(pkg, lens):
    B, Sq, Sk, H = 2, 150, 80, 3
    q, k, v = _qkv(B, Sq, Sk, H, seed=31)
    seq = torch.tensor(lens, dtype=torch.int32)
    out, lse = torch.ops.anima_flat.fa_fwd_k(*_gpu(q, k, v), seq.cuda())
    torch.cuda.synchronize()
    eo, el = ref.attention_lse(q, k, v, seq)
    parity(out, eo, name=f"fa_fwd_k out {lens}")
    parity(lse, el, **LSE_TOL, name=f"fa_fwd_k lse {lens}")
    # Equals plain attention over the first len keys.
    for b, n in enumerate(lens):
        parity(out[b : b + 1], ref.attention_sdpa(q[b : b + 1], k[b : b + 1, :n], v[b : b + 1, :n]),
               name=f"truncated b{b}")


def test_cross_attention_trimmed_matches_padded(pkg):
    """Trimmed attention + padding correction == attention over the zero-padded context."""
    B, Sq, H, S_full = 2, 256, 4, 96
    g = torch.Generator().manual_seed(41)
    q = ref.bf16_normal((B, Sq, H, 128), g)
    lens = torch.tensor([29, 70], dtype=torch.int32)
    k_full = torch.zeros(B, S_full, H, 128)
    v_full = torch.zeros(B, S_full, H, 128)
    for b, n in enumerate(lens.tolist()):
        k_full[b, :n] = ref.bf16_normal((n, H, 128), g)
        v_full[b, :n] = ref.bf16_normal((n, H, 128), g)
    keep = 72  # roundup8(max len)
    ln_pad = torch.log((S_full - lens).float())
    out = pkg.cross_attention_trimmed(
        *_gpu(q, k_full[:, :keep], v_full[:, :keep]), lens.cuda(), ln_pad.cuda()
    )
    torch.cuda.synchronize()
    padded = ref.attention_sdpa(q, k_full, v_full).reshape(B, Sq, H * 128)
    parity(out, padded, name="trimmed vs padded")
    # Same through the two-op path of the reference (fa_fwd_k then ctx_scale).
    o2, l2 = torch.ops.anima_flat.fa_fwd_k(*_gpu(q, k_full[:, :keep], v_full[:, :keep]), lens.cuda())
    y = pkg.ctx_scale(o2, l2, ln_pad.cuda())
    torch.cuda.synchronize()
    parity(y.flatten(2), padded, name="fa_fwd_k + ctx_scale vs padded")


def test_config3_masked_full(pkg):
    """Config 3: B=2, 4096 queries, 512 padded keys, lengths uniform in [32, 512]."""
    g = torch.Generator().manual_seed(1003)
    B, Sq, Sk, H = 2, 4096, 512, 16
    lens = torch.randint(32, 513, (B,), generator=g, dtype=torch.int32)
    x = ref.bf16_normal((B, Sq, H * 128), g)
    w = ref.norm_weight(128, g)
    k = ref.bf16_normal((B, Sk, H, 128), g)
    v = ref.bf16_normal((B, Sk, H, 128), g)
    qd = pkg.head_norm(x.cuda().to(BF), w.cuda(), H, 1e-6)
    out, lse = torch.ops.anima_flat.fa_fwd_k(qd, *_gpu(k, v), lens.cuda())
    torch.cuda.synchronize()
    q = ref.head_norm(x, w, H, 1e-6)
    parity(qd, q, name="config3 head_norm")
    eo, el = ref.attention_lse(q, k, v, lens)
    parity(out, eo, name="config3 masked out")
    parity(lse, el, **LSE_TOL, name="config3 masked lse")


@pytest.mark.parametrize(
    "B,Sq,Sk,H",
    [
        (1, 256, 256, 2),
        (2, 100, 77, 3),  # partial tiles on both sides
        (1, 64, 300, 1),
        (1, 150, 200, 2),  # three query tiles
        (1, 1024, 1024, 4),
    ],
)
def test_attention_backward(pkg, B, Sq, Sk, H):
    q, k, v = _qkv(B, Sq, Sk, H, seed=51 + Sq)
    g = torch.Generator().manual_seed(52)
    dout = ref.bf16_normal((B, Sq, H, 128), g)
    qd, kd, vd = (t.requires_grad_(True) for t in _gpu(q, k, v))
    out = pkg.attention(qd, kd, vd)
    out.backward(dout.to("cuda", BF).reshape(out.shape))
    torch.cuda.synchronize()
    dq, dk, dv = ref.attention_backward(q, k, v, dout)
    parity(qd.grad, dq, name="dq")
    parity(kd.grad, dk, name="dk")
    parity(vd.grad, dv, name="dv")


def _fwd_bwd_grads(pkg, monkeypatch, form, q, k, v, dout):
    _set_form(monkeypatch, form)
    qd, kd, vd = (t.requires_grad_(True) for t in _gpu(q, k, v))
    out = pkg.attention(qd, kd, vd)
    out.backward(dout.to("cuda", BF).reshape(out.shape))
    torch.cuda.synchronize()
    _clear_form(monkeypatch)
    return out, qd.grad.float().cpu(), kd.grad.float().cpu(), vd.grad.float().cpu()


def _rel_l2(a, e):
    return ((a - e).norm() / e.norm().clamp_min(1e-30)).item()


@pytest.mark.parametrize("delta", [0.0, 12.0, 40.0])
def test_backward_after_first_tile_max_forward(pkg, monkeypatch, delta):
    """Training at B >= 2 runs the forward in its first-tile-max form, whose LSE (of the
    bf16-rounded p, with m below the row max) feeds the backward. Forward forced into that
    form, then the backward, against autograd through the oracle.

    delta 0: ordinary rows, the north-star bar on dq, dk and dv. delta 12 (rows on one
    key, in range) and 40 (re-run by the fix-up launch): the hot keys' gradients reach
    magnitudes of 25-70, where the 2e-2 bar is below one bf16 ulp, and the exact dq of a
    row on one key is ~0, so what the backward leaves there (~3e-2: D = rowsum(dO * O) on
    the bf16 O, as in any flash-attention backward) is the same for every forward form.
    There: dk and dv to rel-L2 5e-3, and dq no further from the oracle than after the
    running-max forward (+1e-2)."""
    B, Sq, Sk, H = 2, 300, 2600, 2
    q, k, v = _spiked(B, Sq, Sk, H, delta, [700, 2100], seed=7100 + int(delta))
    g = torch.Generator().manual_seed(7199)
    dout = ref.bf16_normal((B, Sq, H, 128), g)
    out, dq_f, dk_f, dv_f = _fwd_bwd_grads(pkg, monkeypatch, "1w-ftm", q, k, v, dout)
    dq, dk, dv = ref.attention_backward(q, k, v, dout)
    parity(out, ref.attention_sdpa(q, k, v).reshape(out.shape), name=f"out delta={delta}")
    if delta == 0.0:
        parity(dq_f, dq, name="dq")
        parity(dk_f, dk, name="dk")
        parity(dv_f, dv, name="dv")
        return
    _, dq_r, dk_r, dv_r = _fwd_bwd_grads(pkg, monkeypatch, "1w-run", q, k, v, dout)
    for nm, a, e in (("dk", dk_f, dk), ("dv", dv_f, dv)):
        rl = _rel_l2(a, e)
        print(f"[parity] {nm} delta={delta}: rel_l2={rl:.3e} (running-max forward {_rel_l2(dk_r if nm == 'dk' else dv_r, e):.3e})", flush=True)
        assert rl <= 5e-3, f"{nm} delta={delta}: rel_l2 {rl:.3e}"
    err_f = (dq_f - dq).abs().max().item()
    err_r = (dq_r - dq).abs().max().item()
    print(f"[parity] dq delta={delta}: max_abs={err_f:.3e} (running-max forward {err_r:.3e})", flush=True)
    assert err_f <= err_r + 1e-2, f"dq delta={delta}: {err_f:.3e} against {err_r:.3e}"


def test_backward_deterministic(pkg):
    q, k, v = _qkv(1, 384, 384, 2, seed=61)
    dout = torch.randn(1, 384, 2, 128).to("cuda", BF)
    qd, kd, vd = _gpu(q, k, v)
    out, lse = torch.ops.anima_flat.fa_fwd(qd, kd, vd)
    g1 = torch.ops.anima_flat.fa_bwd(dout, qd, kd, vd, out, lse)
    g2 = torch.ops.anima_flat.fa_bwd(dout, qd, kd, vd, out, lse)
    torch.cuda.synchronize()
    for a, b in zip(g1, g2):
        assert torch.equal(a, b)


def test_softmax_scale_is_inverse_sqrt_hd(pkg):
    """One key: output = v regardless of scale; two equal keys: average of values."""
    B, Sq, H = 1, 64, 1
    g = torch.Generator().manual_seed(71)
    q = ref.bf16_normal((B, Sq, H, 128), g)
    k = ref.bf16_normal((B, 2, H, 128), g)
    k[:, 1] = k[:, 0]
    v = ref.bf16_normal((B, 2, H, 128), g)
    out = pkg.attention(*_gpu(q, k, v)).view(B, Sq, H, 128)
    torch.cuda.synchronize()
    exp = ((v[:, 0] + v[:, 1]) / 2)[:, None].expand(B, Sq, H, 128)
    parity(out, exp, max_abs=1e-2, rel_l2=4e-3, name="equal keys")
    assert math.isclose(1 / math.sqrt(128), 0.08838834764831845)


def _random_shapes(n, seed):
    g = torch.Generator().manual_seed(seed)
    out = []
    for _ in range(n):
        B = int(torch.randint(1, 4, (1,), generator=g))
        H = int(torch.randint(1, 6, (1,), generator=g))
        Sq = int(torch.randint(1, 700, (1,), generator=g))
        Sk = int(torch.randint(1, 700, (1,), generator=g))
        out.append((B, Sq, Sk, H))
    return out


@pytest.mark.parametrize("B,Sq,Sk,H", _random_shapes(8, seed=2024) + [(1, 1, 1, 1), (2, 31, 1, 3)])
def test_random_shapes_forward_backward(pkg, B, Sq, Sk, H):
    """Seeded random sizes (partial query blocks, waves and key tiles everywhere), K and V as
    strided views of one [B, Sk, 2, H, 128] buffer, forward and backward against the oracle."""
    g = torch.Generator().manual_seed(B * 1000003 + Sq * 1009 + Sk * 7 + H)
    q = ref.bf16_normal((B, Sq, H, 128), g)
    kv = ref.bf16_normal((B, Sk, 2, H, 128), g)
    k, v = kv[:, :, 0], kv[:, :, 1]
    dout = ref.bf16_normal((B, Sq, H, 128), g)
    qd = q.to("cuda", BF).requires_grad_(True)
    kvd = kv.to("cuda", BF).requires_grad_(True)
    out = pkg.attention(qd, kvd[:, :, 0], kvd[:, :, 1])
    out.backward(dout.to("cuda", BF).reshape(out.shape))
    torch.cuda.synchronize()
    tag = f"B{B} Sq{Sq} Sk{Sk} H{H}"
    parity(out, ref.attention_sdpa(q, k, v).reshape(B, Sq, H * 128), name=f"fwd {tag}")
    dq, dk, dv = ref.attention_backward(q, k, v, dout)
    if Sk == 1:
        # One key: P = 1 and dP = D, so dQ (and dK) are exactly 0 and a relative
        # norm is undefined; the bar is max-abs alone.
        assert qd.grad.abs().max().item() <= 1e-5 and kvd.grad[:, :, 0].abs().max().item() <= 1e-5
        # dV = sum of dO over all queries (P = 1): values of ~10, where one bf16
        # rounding step alone is 2^-4; the max-abs bar is bf16's half-ulp at that size.
        bar = max(2e-2, dv.abs().max().item() * 2.0**-8)
        parity(kvd.grad[:, :, 1], dv, max_abs=bar, name=f"dv {tag}")
    else:
        parity(qd.grad, dq, name=f"dq {tag}")
        parity(kvd.grad[:, :, 0], dk, name=f"dk {tag}")
        parity(kvd.grad[:, :, 1], dv, name=f"dv {tag}")


@pytest.mark.parametrize("B,S,H", [(1, 16384, 2), (2, 12288, 1)])
def test_long_sequence_sampled_rows(pkg, B, S, H):
    """Long sequences (hundreds of key tiles; the split-key path for the last round): the
    full kernel against the oracle on 96 sampled query rows of every (batch, head)."""
    g = torch.Generator().manual_seed(S + H)
    q, k, v = _qkv(B, S, S, H, seed=S + B)
    out, lse = torch.ops.anima_flat.fa_fwd(*_gpu(q, k, v))
    torch.cuda.synchronize()
    rows = torch.randperm(S, generator=g)[:96].sort().values
    eo, el = ref.attention_lse(q[:, rows], k, v)
    parity(out[:, rows].reshape(B, 96, H, 128), eo, name=f"long S{S} B{B} H{H}")
    parity(lse[:, :, rows], el, **LSE_TOL, name=f"long lse S{S}")


def test_long_sequence_backward_sampled_rows(pkg):
    """Backward at 16384 tokens (256 key tiles per dQ block, 128 query tiles per dK/dV block):
    dQ on 64 sampled query rows and dK/dV on 64 sampled key rows against the chunked
    closed-form oracle."""
    B, S, H = 1, 16384, 1
    q, k, v = _qkv(B, S, S, H, seed=16385)
    g = torch.Generator().manual_seed(16386)
    dout = ref.bf16_normal((B, S, H, 128), g)
    qd, kd, vd = (t.requires_grad_(True) for t in _gpu(q, k, v))
    out = pkg.attention(qd, kd, vd)
    out.backward(dout.to("cuda", BF).reshape(out.shape))
    torch.cuda.synchronize()
    qrows = torch.randperm(S, generator=g)[:64].sort().values
    krows = torch.cat([torch.randperm(S - 1, generator=g)[:63].sort().values, torch.tensor([S - 1])])
    dq, dk, dv = ref.attention_backward_rows(q, k, v, dout, qrows, krows)
    parity(qd.grad[:, qrows], dq, name="long dq")
    parity(kd.grad[:, krows], dk, name="long dk")
    parity(vd.grad[:, krows], dv, name="long dv")


def test_cross_attention_backward_training_shape(pkg):
    """LoRA training's cross-attention backward: fa_bwd at B=2, Sq=4096, Sk=512 over
    the untrimmed, zero-padded text context (src/model.py:326 -> src/attention.py
    :143-146, :118-120; the context is not trimmed under grad). Projecting a zero
    context row and RMS-normalising its key gives zero K and V rows, which still
    take part in the softmax (score 0). dQ on 64 sampled query rows of each item,
    dK/dV on 64 sampled key rows that include padded ones, against the chunked
    closed-form oracle."""
    B, Sq, Sk, H = 2, 4096, 512, 16
    q, k, v = _qkv(B, Sq, Sk, H, seed=4099)
    for b, n in enumerate((58, 322)):
        k[b, n:] = 0
        v[b, n:] = 0
    g = torch.Generator().manual_seed(4100)
    dout = ref.bf16_normal((B, Sq, H, 128), g)
    qd, kd, vd = (t.requires_grad_(True) for t in _gpu(q, k, v))
    out = pkg.attention(qd, kd, vd)
    out.backward(dout.to("cuda", BF).reshape(out.shape))
    torch.cuda.synchronize()
    qrows = torch.randperm(Sq, generator=g)[:64].sort().values
    krows = torch.cat([torch.tensor([0, 57, 58, 321, 322, Sk - 1]),
                       torch.randperm(Sk, generator=g)[:58]]).unique().sort().values
    dq, dk, dv = ref.attention_backward_rows(q, k, v, dout, qrows, krows)
    parity(qd.grad[:, qrows], dq, name="cross bwd dq")
    parity(kd.grad[:, krows], dk, name="cross bwd dk")
    parity(vd.grad[:, krows], dv, name="cross bwd dv")
    eo = ref.attention_lse(q[:, qrows], k, v)[0]
    parity(out.reshape(B, Sq, H, 128)[:, qrows], eo, name="cross fwd (sampled rows)")


@pytest.mark.parametrize("kernel", ["pp", "1w", "1w-ftm", "1w-run"])
@pytest.mark.parametrize(
    "B,Sq,Sk,H,lens",
    [
        (1, 1024, 1024, 16, None),  # config 1: 64 work items, split over key ranges
        (2, 4096, 512, 4, [58, 322]),  # config 3's masked cross-attention
        (1, 300, 777, 3, None),  # ragged: partial query and key tiles
        (2, 700, 2500, 2, [2500, 1]),  # one key; a key length past 2048
        (1, 4096, 4096, 2, None),  # long: 64 key tiles
    ],
)
def test_both_forward_kernels(pkg, monkeypatch, kernel, B, Sq, Sk, H, lens):
    """aa_attn_fwd runs the two-group kernel up to 2048 keys and the one-wave-per-SIMD
    kernel beyond (AA_FWD_KERNEL forces one), the latter in its first-tile-max form
    (with the fix-up launch) from about a round of 64-tile work items on and with the
    running max below (AA_FWD_FIRST_TILE_MAX forces one); each is held to the oracle
    on every shape, with and without key lengths, and its LSE."""
    q, k, v = _qkv(B, Sq, Sk, H, seed=9000 + Sq + Sk + H)
    seq = torch.tensor(lens, dtype=torch.int32) if lens is not None else None
    _set_form(monkeypatch, kernel)
    qd, kd, vd = _gpu(q, k, v)
    if seq is None:
        out, lse = torch.ops.anima_flat.fa_fwd(qd, kd, vd)
    else:
        out, lse = torch.ops.anima_flat.fa_fwd_k(qd, kd, vd, seq.to("cuda"))
    torch.cuda.synchronize()
    _clear_form(monkeypatch)
    eo, el = ref.attention_lse(q, k, v, seq)
    tag = f"{kernel} B{B} Sq{Sq} Sk{Sk} H{H} lens={lens}"
    parity(out, eo, name=tag)
    parity(lse, el, **LSE_TOL, name=f"lse {tag}")


@pytest.mark.parametrize("kernel", ["1w", "2role"])
@pytest.mark.parametrize(
    "B,Sq,Sk,H",
    [
        (2, 100, 77, 3),  # partial query and key tiles, keys past Sk in every wave
        (1, 64, 300, 1),  # one query tile
        (1, 2048, 256, 4),  # 8 key blocks: the query range split over 4 workgroups
        (1, 1000, 300, 2),  # split with a partial last query tile
        (1, 1024, 1024, 4),
    ],
)
def test_both_dkdv_kernels(pkg, monkeypatch, kernel, B, Sq, Sk, H):
    """aa_attn_bwd runs the one-wave-per-SIMD dK/dV kernel unless AA_DKDV_KERNEL=2role
    picks the two-role one; each is held to the oracle on every shape, with and
    without the query split and its combine pass."""
    q, k, v = _qkv(B, Sq, Sk, H, seed=9200 + Sq + Sk + H)
    g = torch.Generator().manual_seed(9201)
    dout = ref.bf16_normal((B, Sq, H, 128), g)
    qd, kd, vd = _gpu(q, k, v)
    out, lse = torch.ops.anima_flat.fa_fwd(qd, kd, vd)
    monkeypatch.setenv("AA_DKDV_KERNEL", kernel)
    dqg, dkg, dvg = torch.ops.anima_flat.fa_bwd(dout.to("cuda", BF), qd, kd, vd, out, lse)
    torch.cuda.synchronize()
    monkeypatch.delenv("AA_DKDV_KERNEL")
    dq, dk, dv = ref.attention_backward(q, k, v, dout)
    tag = f"{kernel} B{B} Sq{Sq} Sk{Sk} H{H}"
    parity(dqg, dq, name=f"dq {tag}")
    parity(dkg, dk, name=f"dk {tag}")
    parity(dvg, dv, name=f"dv {tag}")


def test_dkdv_kernel_env_rejects_unknown_value(pkg, monkeypatch):
    q, k, v = _gpu(*_qkv(1, 64, 64, 1, seed=9300))
    out, lse = torch.ops.anima_flat.fa_fwd(q, k, v)
    monkeypatch.setenv("AA_DKDV_KERNEL", "zz")
    with pytest.raises(ValueError, match="AA_DKDV_KERNEL"):
        torch.ops.anima_flat.fa_bwd(torch.ones_like(q), q, k, v, out, lse)


def test_forward_kernel_env_rejects_unknown_value(pkg, monkeypatch):
    q, k, v = _gpu(*_qkv(1, 64, 64, 1, seed=9100))
    monkeypatch.setenv("AA_FWD_KERNEL", "zz")
    with pytest.raises(ValueError, match="AA_FWD_KERNEL"):
        torch.ops.anima_flat.fa_fwd(q, k, v)
