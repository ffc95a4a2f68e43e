"""GPU parity of the paths the product runs end to end, at their real sizes.

* The config-2 chain exactly as `bench.py` times it: no-grad `qkv_norm_rope`
  (q, k written, V returned as a strided view of qkv, row stride 3*H*hd), then
  `anima_flat::fa_fwd_nolse` on those tensors (src/kernels/rope.py:616-645,
  src/attention.py:63-66, src/model.py:308-330).
* The prologue at config-4 sizes (4a: B=16 x 4096 tokens; 4b: 9216 tokens on a
  96x96 grid).
* `use_fa4` on the GPU (src/attention.py:21-40) and its env override.
* `Context.attend` in both branches (src/model.py:106-119), including the
  on-device lengths of `context_lengths`.

Bar: max-abs 2e-2 and relative L2 5e-3 against the fp32 CPU oracle; where a
result is produced by the same kernel on the same inputs, equality is exact.
"""

from __future__ import annotations

import pytest
import torch

from conftest import parity
from oracle import attn_oracle as ref

pytestmark = pytest.mark.gpu

BF = torch.bfloat16
DEV = "cuda:0"


def _prologue(pkg, inp, H, eps):
    with torch.no_grad():
        return pkg.qkv_norm_rope(
            inp["qkv"].to(DEV, BF), inp["q_weight"].to(DEV), inp["k_weight"].to(DEV),
            inp["cos"].to(DEV), inp["sin"].to(DEV), H, eps,
        )


def test_bench_chain_config2_full(pkg):
    """The bench's input and op: config 2 (B=1, 4096 tokens, 16 heads), seed 1002."""
    B, S, H, eps = 1, 4096, 16, 1e-6
    inp = ref.prologue_inputs(B, S, H, 128, seed=1002)
    q, k, v = _prologue(pkg, inp, H, eps)
    assert not v.is_contiguous() and v.stride(1) == 3 * H * 128  # V read in place from qkv
    with torch.no_grad():
        out = torch.ops.anima_flat.fa_fwd_nolse(q, k, v)
        out_api = pkg.attention(q, k, v)
    torch.cuda.synchronize()
    rq, rk, rv = ref.qkv_norm_rope(inp["qkv"], inp["q_weight"], inp["k_weight"], inp["cos"], inp["sin"], H, eps)
    parity(q, rq, name="config2 chain q")
    parity(k, rk, name="config2 chain k")
    assert torch.equal(v.float().cpu(), rv)
    # Attention of the GPU's own q, k (isolates the forward) and of the oracle's.
    exp = ref.attention_sdpa(q.float().cpu(), k.float().cpu(), rv)
    parity(out, exp, name="config2 chain attention")
    parity(out, ref.attention_sdpa(rq, rk, rv), name="config2 chain vs oracle prologue")
    assert torch.equal(out_api, out.flatten(2))


@pytest.mark.parametrize("B,S,check", [(16, 4096, (0, 7, 15)), (1, 9216, (0,))])
def test_prologue_config4_sizes(pkg, B, S, check):
    """Config 4a (B=16 x 4096) and 4b (9216 tokens, 96x96 rope grid); eps 1e-6.
    Tokens are independent, so the listed batch items are compared in full."""
    H, eps = 16, 1e-6
    inp = ref.prologue_inputs(B, S, H, 128, seed=1040 + B)
    q, k, v = _prologue(pkg, inp, H, eps)
    torch.cuda.synchronize()
    assert q.shape == (B, S, H, 128) and v.stride(1) == 3 * H * 128
    for b in check:
        sub = inp["qkv"][b : b + 1]
        rq, rk, rv = ref.qkv_norm_rope(sub, inp["q_weight"], inp["k_weight"], inp["cos"], inp["sin"], H, eps)
        parity(q[b : b + 1], rq, name=f"config4 S={S} batch {b} q")
        parity(k[b : b + 1], rk, name=f"config4 S={S} batch {b} k")
        mism = (q[b : b + 1].float().cpu() != rq).float().mean().item()
        assert mism < 1e-3, f"{mism:.2e} of q elements differ from the rounded oracle"
        assert torch.equal(v[b : b + 1].float().cpu(), rv)


def test_use_fa4_on_gpu(pkg, monkeypatch):
    """True for bf16 tensors on a gfx950 GPU; False for other dtypes, CPU tensors and
    under ANIMA_FLAT_ATTENTION=sdpa (read at call time)."""
    t = torch.zeros(1, 8, 1, 128, dtype=BF, device=DEV)
    assert "gfx950" in torch.cuda.get_device_properties(0).gcnArchName
    monkeypatch.delenv("ANIMA_FLAT_ATTENTION", raising=False)
    assert pkg.use_fa4(t) is True
    assert pkg.use_fa4(t.float()) is False
    assert pkg.use_fa4(t.cpu()) is False
    monkeypatch.setenv("ANIMA_FLAT_ATTENTION", "sdpa")
    assert pkg.use_fa4(t) is False
    monkeypatch.setenv("ANIMA_FLAT_ATTENTION", "fa4")
    assert pkg.use_fa4(t) is True


def _cross_inputs(B, Sq, Sk, H, seed):
    g = torch.Generator().manual_seed(seed)
    q = ref.bf16_normal((B, Sq, H, 128), g)
    kv = [(ref.bf16_normal((B, Sk, H, 128), g), ref.bf16_normal((B, Sk, H, 128), g)) for _ in range(2)]
    return q, kv


def test_context_attend_untrimmed(pkg):
    """Context(kv).attend(layer, q) = attention(q, k_layer, v_layer) (model.py:116-117)."""
    B, Sq, Sk, H = 2, 512, 512, 4
    q, kv = _cross_inputs(B, Sq, Sk, H, seed=301)
    kvd = [(k.to(DEV, BF), v.to(DEV, BF)) for k, v in kv]
    ctx = pkg.Context(kvd)
    qd = q.to(DEV, BF)
    with torch.no_grad():
        outs = [ctx.attend(layer, qd) for layer in (0, 1)]
        direct = [pkg.attention(qd, k, v) for k, v in kvd]
    torch.cuda.synchronize()
    for layer in (0, 1):
        assert outs[layer].shape == (B, Sq, H * 128)
        assert torch.equal(outs[layer], direct[layer])
        exp = ref.attention_sdpa(q, *kv[layer]).reshape(B, Sq, H * 128)
        parity(outs[layer], exp, name=f"attend untrimmed layer {layer}")


def test_context_attend_trimmed(pkg):
    """Trimmed branch (model.py:118-119): cross_attention_trimmed with the trim's lengths,
    both from trim_context (sliced K/V) and from context_lengths (whole K/V, lengths
    on the device); both equal the oracle's masked attention + padding correction."""
    B, Sq, S, H, C = 2, 1024, 512, 4, 256
    lens = torch.tensor([58, 322])
    g = torch.Generator().manual_seed(311)
    ctx = ref.bf16_normal((B, S, C), g)
    for b in range(B):
        ctx[b, lens[b]:] = 0.0
    q, kv = _cross_inputs(B, Sq, S, H, seed=312)
    ctxd = ctx.to(DEV, BF)
    sliced, seqused, ln_pad = pkg.trim_context(ctxd)
    keep = sliced.shape[1]
    assert keep == 328 and seqused.tolist() == lens.tolist()
    dev_seqused, dev_ln_pad = pkg.context_lengths(ctxd)
    assert torch.equal(dev_seqused, seqused)
    assert torch.allclose(dev_ln_pad, ln_pad, rtol=2**-23, atol=0)  # log of an integer, within 1 ulp
    kvd = [(k.to(DEV, BF), v.to(DEV, BF)) for k, v in kv]
    qd = q.to(DEV, BF)
    trimmed = pkg.Context([(k[:, :keep], v[:, :keep]) for k, v in kvd], seqused, ln_pad)
    ondev = pkg.Context(kvd, dev_seqused, dev_ln_pad)
    with torch.no_grad():
        a = [trimmed.attend(layer, qd) for layer in (0, 1)]
        b = [ondev.attend(layer, qd) for layer in (0, 1)]
        direct = pkg.cross_attention_trimmed(qd, kvd[1][0][:, :keep], kvd[1][1][:, :keep], seqused, ln_pad)
    torch.cuda.synchronize()
    assert torch.equal(a[1], direct)
    for layer in (0, 1):
        assert a[layer].shape == (B, Sq, H * 128)
        k, v = kv[layer]
        exp = ref.cross_attention_trimmed(q, k, v, lens.to(torch.int32), torch.log((S - lens).float()))
        exp = exp.reshape(B, Sq, H * 128)
        parity(a[layer], exp, name=f"attend trimmed layer {layer}")
        parity(b[layer], exp, name=f"attend on-device lengths layer {layer}")
