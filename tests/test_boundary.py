"""CPU tests of the drop-in boundary: the C ABI library and the Python layer.

No kernel runs here: the C-ABI calls below fail argument validation before any
HIP call, and the Python ops are exercised through their fake (meta)
implementations.
"""

from __future__ import annotations

import ctypes
import math
import re
import subprocess
import sys
from pathlib import Path

import pytest
import torch

import __graft_entry__
from oracle import attn_oracle as ref

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "anima_attn.h"


@pytest.fixture(scope="module")
def lib(pkg):
    if not pkg._lib.LIB_PATH.exists():
        pytest.skip("libanima_attn.so not built (run __graft_entry__.build())")
    return pkg._lib.lib()


def _declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(aa_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_entry_points():
    names = _declared_functions()
    for expected in (
        "aa_abi_version",
        "aa_last_error",
        "aa_qkv_norm_rope_fwd",
        "aa_qkv_norm_rope_bwd",
        "aa_head_norm_fwd",
        "aa_head_norm_bwd",
        "aa_attn_fwd",
        "aa_attn_fwd_workspace",
        "aa_attn_bwd",
        "aa_attn_bwd_workspace",
        "aa_ctx_scale_fwd",
        "aa_ctx_scale_bwd",
    ):
        assert expected in names


def test_library_exports_every_declared_symbol(lib):
    for name in _declared_functions():
        assert hasattr(lib, name), f"{name} missing from libanima_attn.so"
    out = subprocess.run(["nm", "-D", "--defined-only", str(ROOT / "anima-flat_amd" / "libanima_attn.so")],
                         capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\bT (aa_[a-z0-9_]+)", out))
    assert set(_declared_functions()) <= exported


def test_python_binding_covers_the_header(pkg):
    assert set(pkg._lib.EXPORTED) == set(_declared_functions())


def test_abi_version(pkg, lib):
    assert lib.aa_abi_version() == pkg._lib.ABI_VERSION


def test_structs_match_header_field_order(pkg):
    text = HEADER.read_text()
    for struct, cls in (("aa_attn_fwd_args", pkg._lib.AttnFwdArgs), ("aa_attn_bwd_args", pkg._lib.AttnBwdArgs)):
        body = re.search(r"typedef struct %s \{(.*?)\} %s;" % (struct, struct), text, re.S).group(1)
        body = re.sub(r"/\*.*?\*/", "", body, flags=re.S)
        types = {"const", "void", "float", "int", "int32_t", "int64_t", "size_t"}
        fields = [tok.split("[")[0] for decl in body.split(";")
                  for tok in re.findall(r"[A-Za-z_][A-Za-z0-9_]*(?:\[\d+\])?", decl)
                  if tok.split("[")[0] not in types]
        assert [f[0] for f in cls._fields_] == fields


def test_workspace_sizes(lib):
    # one 1 KB stats record per 64-query tile, per (batch, head)
    assert lib.aa_attn_bwd_workspace(2, 100, 77, 3, 128) == 2 * 3 * 2 * 1024
    assert lib.aa_attn_bwd_workspace(1, 0, 77, 3, 128) == 0
    # weight-gradient partials: one [2][128] fp32 record per block of 64
    # (token, head) items, one [128] record per 128 items for head_norm
    assert lib.aa_qkv_norm_rope_bwd_workspace(1, 4096, 16, 128) == 1024 * 2 * 128 * 4
    assert lib.aa_head_norm_bwd_workspace(2, 9, 5, 128) == 1 * 128 * 4
    assert lib.aa_head_norm_bwd_workspace(2, 65, 1, 128) == 2 * 128 * 4
    assert lib.aa_head_norm_bwd_workspace(0, 65, 1, 128) == 0
    # one int32 per 32 context rows per item
    assert lib.aa_context_lengths_workspace(3, 77) == 3 * 3 * 4
    assert lib.aa_context_lengths_workspace(0, 77) == 0


def test_invalid_arguments_fail_before_any_launch(pkg, lib):
    L = pkg._lib
    assert lib.aa_attn_fwd(None, None) == L.AA_EINVAL
    assert "null args" in lib.aa_last_error().decode()
    a = L.AttnFwdArgs()
    a.B, a.Sq, a.Sk, a.H, a.hd, a.dtype, a.softmax_scale = 1, 4, 4, 1, 64, 0, 0.125
    assert lib.aa_attn_fwd(ctypes.byref(a), None) == L.AA_EUNSUPPORTED
    assert "head_dim" in lib.aa_last_error().decode()
    a.hd, a.dtype = 128, 1
    assert lib.aa_attn_fwd(ctypes.byref(a), None) == L.AA_EUNSUPPORTED
    a.dtype = 0
    assert lib.aa_attn_fwd(ctypes.byref(a), None) == L.AA_EINVAL  # null tensors
    b = L.AttnBwdArgs()
    assert lib.aa_attn_bwd(None, None, 0, None) == L.AA_EINVAL
    b.B, b.Sq, b.Sk, b.H, b.hd, b.dtype = 1, 4, 4, 1, 128, 0
    assert lib.aa_attn_bwd(ctypes.byref(b), None, 0, None) == L.AA_EINVAL
    assert lib.aa_qkv_norm_rope_fwd(None, None, None, None, None, None, None, None, 1, 4, 2, 128, 1e-6, 0, None) == L.AA_EINVAL
    assert lib.aa_head_norm_fwd(None, None, None, 1, 4, 2, 96, 1e-6, 0, None) == L.AA_EUNSUPPORTED
    proj = lambda H, hd, dtype, B=1, rs=256: lib.aa_qkv_proj_norm_rope(
        None, rs, None, None, None, None, None, None, None, None, B, 4, H, hd, 1e-6, dtype, None)
    assert proj(2, 96, 0) == L.AA_EUNSUPPORTED  # head_dim
    assert proj(2, 128, 1) == L.AA_EUNSUPPORTED  # dtype
    assert proj(65, 128, 0) == L.AA_EINVAL  # H > 64
    assert proj(2, 128, 0) == L.AA_EINVAL  # null pointers
    assert proj(2, 128, 0, B=0) == L.AA_OK  # no tokens: nothing to do
    assert proj(2, 128, 0, rs=(1 << 27) + 8) == L.AA_EUNSUPPORTED  # 32-bit DMA offsets
    assert "row stride" in lib.aa_last_error().decode()
    xq = lambda hd, K, B=1: lib.aa_proj_head_norm(None, 256, None, K, None, None, B, 4, 2, hd, 1e-6, 0, None)
    assert xq(96, 256) == L.AA_EUNSUPPORTED  # head_dim
    assert xq(128, 80) == L.AA_EUNSUPPORTED  # K % 32
    assert xq(128, 256) == L.AA_EINVAL  # null pointers
    assert xq(128, 256, B=0) == L.AA_OK
    xkv = lambda K, rs=1024: lib.aa_kv_proj_norm(None, rs, None, K, None, None, None, 1, 4, 2, 128, 1e-6, 0, None)
    assert xkv(1000) == L.AA_EUNSUPPORTED  # K % 32
    assert xkv(1024) == L.AA_EINVAL  # null pointers
    assert "kv_proj_norm" in lib.aa_last_error().decode()
    assert lib.aa_ctx_scale_fwd(None, None, None, None, 1, 4, 2, 128, 3, None) == L.AA_EUNSUPPORTED
    assert lib.aa_context_lengths(None, 1, 8, 8, 64, 8, 3, None, None, None, 0, None) == L.AA_EUNSUPPORTED
    assert lib.aa_context_lengths(None, 1, 8, 8, 64, 8, 2, None, None, None, 0, None) == L.AA_EINVAL
    assert lib.aa_rowquant(None, 4, 12, 0, None, None, 0, None) == L.AA_EUNSUPPORTED  # K % 8
    assert lib.aa_rowquant(None, 4, 16384, 0, None, None, 0, None) == L.AA_EUNSUPPORTED
    assert lib.aa_rowquant(None, 4, 16, 0, None, None, 0, None) == L.AA_EINVAL  # null
    with pytest.raises(ValueError):
        L.check(L.AA_EINVAL, "x")
    with pytest.raises(RuntimeError):
        L.check(L.AA_EHIP, "x")


def test_cpu_tensors_are_rejected(pkg, fp8, proj):
    q = torch.zeros(1, 4, 1, 128, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="CUDA tensors required"):
        pkg.attention(q, q, q)
    with pytest.raises(ValueError, match="CUDA tensors required"):
        pkg.cross_attention_trimmed(q, q, q, torch.tensor([4], dtype=torch.int32), torch.tensor([0.0]))
    qkv = torch.zeros(1, 4, 3 * 128, dtype=torch.bfloat16)
    w = torch.ones(128)
    cos = torch.ones(4, 64)
    with pytest.raises(ValueError, match="CUDA tensors required"):
        pkg.qkv_norm_rope(qkv, w, w, cos, cos, 1)
    with pytest.raises(ValueError, match="CUDA tensors required"):
        pkg.head_norm(torch.zeros(1, 4, 128, dtype=torch.bfloat16), w, 1)
    with pytest.raises(ValueError, match="CUDA tensors required"):
        pkg.ctx_scale(q, torch.zeros(1, 1, 4), torch.zeros(1))
    with pytest.raises(ValueError, match="CUDA tensors required"):
        pkg.context_lengths(torch.zeros(1, 4, 8, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="CUDA tensors required"):
        fp8.rowquant(torch.zeros(1, 4, 8, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="CUDA"):
        proj.qkv_proj_norm_rope(torch.zeros(1, 4, 256, dtype=torch.bfloat16),
                               torch.zeros(768, 256, dtype=torch.bfloat16), torch.ones(128),
                               torch.ones(128), torch.zeros(4, 64), torch.zeros(4, 64), 2)
    assert pkg.use_fa4(q) is False


def test_ops_are_registered_with_reference_names(pkg, fp8, proj):
    for name in ("fa_fwd", "fa_fwd_nolse", "fa_fwd_k", "fa_bwd", "qkv_norm_rope", "qkv_norm_rope_v",
                 "qkv_norm_rope_bwd", "head_norm", "head_norm_bwd", "ctx_scale", "ctx_scale_bwd",
                 "rowquant"):
        assert hasattr(torch.ops.anima_flat, name), name
    # Ops with no counterpart in the reference live in their own namespace.
    for name in ("fa_fwd_k_ctx", "qkv_proj_norm_rope"):
        assert hasattr(torch.ops.anima_flat_amd, name), name
        assert not hasattr(torch.ops.anima_flat, name), name


_STUB = """
import sys, torch
sys.path.insert(0, {root!r})

@torch.library.custom_op("anima_flat::{name}", mutates_args=())
def stub(x: torch.Tensor, flag: bool) -> tuple[torch.Tensor, torch.Tensor]:
    return x.clone().fill_(7.0), x.new_zeros(1)

import __graft_entry__
"""


def _run_py(code: str) -> subprocess.CompletedProcess:
    return subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300,
                          cwd=ROOT)


def test_package_leaves_foreign_rowquant_alone():
    """The reference's src/kernels/fp8.py registers anima_flat::rowquant; importing this
    package must not replace it, and importing the opt-in module must raise, not re-bind."""
    code = _STUB.format(root=str(ROOT), name="rowquant") + """
amd = __graft_entry__.load_package()
assert not hasattr(amd, "rowquant")
x = torch.zeros(2, 3)
assert torch.equal(torch.ops.anima_flat.rowquant(x, False)[0], torch.full((2, 3), 7.0))
try:
    import anima_flat_amd.kernels.fp8  # noqa: F401
except RuntimeError as e:
    assert "anima_flat::rowquant is already registered" in str(e), e
else:
    raise AssertionError("second registration of anima_flat::rowquant did not raise")
assert torch.equal(torch.ops.anima_flat.rowquant(x, False)[0], torch.full((2, 3), 7.0))
print("ok")
"""
    r = _run_py(code)
    assert r.returncode == 0 and r.stdout.strip().endswith("ok"), r.stdout + r.stderr


def test_package_refuses_to_rebind_reference_attention_op():
    """With the reference's src/attention.py imported first (anima_flat::fa_fwd registered),
    importing the package raises instead of silently taking the name over."""
    code = _STUB.format(root=str(ROOT), name="fa_fwd") + """
try:
    __graft_entry__.load_package()
except RuntimeError as e:
    assert "anima_flat::fa_fwd is already registered" in str(e), e
else:
    raise AssertionError("package import re-bound anima_flat::fa_fwd")
x = torch.zeros(2, 3)
assert torch.equal(torch.ops.anima_flat.fa_fwd(x, False)[0], torch.full((2, 3), 7.0))
print("ok")
"""
    r = _run_py(code)
    assert r.returncode == 0 and r.stdout.strip().endswith("ok"), r.stdout + r.stderr


def test_fake_shapes_on_meta_tensors(pkg, fp8, proj):
    B, Sq, Sk, H = 2, 40, 24, 3
    q = torch.empty(B, Sq, H, 128, dtype=torch.bfloat16, device="meta")
    k = torch.empty(B, Sk, H, 128, dtype=torch.bfloat16, device="meta")
    out, lse = torch.ops.anima_flat.fa_fwd(q, k, k)
    assert out.shape == q.shape and lse.shape == (B, H, Sq) and lse.dtype == torch.float32
    assert torch.ops.anima_flat.fa_fwd_nolse(q, k, k).shape == q.shape
    seq = torch.empty(B, dtype=torch.int32, device="meta")
    out, lse = torch.ops.anima_flat.fa_fwd_k(q, k, k, seq)
    assert out.shape == q.shape and lse.shape == (B, H, Sq)
    dq, dk, dv = torch.ops.anima_flat.fa_bwd(q, q, k, k, q, lse)
    assert dq.shape == q.shape and dk.shape == k.shape and dv.shape == k.shape
    qkv = torch.empty(B, Sq, 3 * H * 128, dtype=torch.bfloat16, device="meta")
    w = torch.empty(128, device="meta")
    cos = torch.empty(Sq, 64, device="meta")
    qq, kk = torch.ops.anima_flat.qkv_norm_rope(qkv, w, w, cos, cos, H, 1e-6)
    assert qq.shape == kk.shape == (B, Sq, H, 128)
    qq, kk, vv = torch.ops.anima_flat.qkv_norm_rope_v(qkv, w, w, cos, cos, H, 1e-6)
    assert vv.shape == (B, Sq, H, 128)
    x = torch.empty(B, Sq, H * 128, dtype=torch.bfloat16, device="meta")
    assert torch.ops.anima_flat.head_norm(x, w, H, 1e-6).shape == (B, Sq, H, 128)
    y = torch.ops.anima_flat.ctx_scale(q, lse, torch.empty(B, device="meta"))
    assert y.shape == q.shape
    x = torch.empty(B, Sq, 2048, dtype=torch.bfloat16, device="meta")
    qx, sx = torch.ops.anima_flat.rowquant(x, False)
    assert qx.shape == x.shape and qx.dtype == torch.float8_e4m3fn and sx.shape == (B * Sq, 1)
    hid = torch.empty(B, Sq, H * 128, dtype=torch.bfloat16, device="meta")
    wq = torch.empty(3 * H * 128, H * 128, dtype=torch.bfloat16, device="meta")
    outs = torch.ops.anima_flat_amd.qkv_proj_norm_rope(hid, wq, w, w, cos, cos, H, 1e-6)
    assert all(t.shape == (B, Sq, H, 128) and t.dtype == torch.bfloat16 for t in outs)


def test_rope_tables_bit_identical_to_oracle(pkg):
    for h, w, scale in ((32, 32, (1.0, 1.0)), (64, 64, (4.0, 4.0)), (3, 5, (1.0, 1.0))):
        c, s = pkg.rope_tables(h, w, 128, "cpu", scale)
        rc, rs = ref.rope_tables(h, w, 128, scale)
        assert torch.equal(c, rc) and torch.equal(s, rs)


def test_trim_context_bookkeeping(pkg):
    ctx = torch.zeros(3, 20, 4)
    ctx[0, :5] = 1.0
    ctx[1, :13] = 1.0
    ctx[1, 7] = 0.0  # interior zero row does not end the sequence
    trimmed, seqused, ln_pad = pkg.trim_context(ctx)  # item 2 all-zero -> length 1
    assert seqused.tolist() == [5, 13, 1] and seqused.dtype == torch.int32
    assert trimmed.shape == (3, 16, 4)  # roundup8(13)
    torch.testing.assert_close(ln_pad, torch.log(torch.tensor([15.0, 7.0, 19.0])))
    full = torch.ones(1, 8, 2)
    t2, s2, l2 = pkg.trim_context(full)
    assert t2.shape[1] == 8 and s2.tolist() == [8] and math.isinf(l2.item()) and l2.item() < 0


def test_projection_row_launches(proj):
    """The fused projections hand B * S input rows to the C ABI at one row
    stride: uniform rows go in one launch (for B == 1 whatever the batch
    stride), a sequence-trimmed context view (src/model.py:251) in one launch
    per batch item, each item's rows at the view's row stride."""
    plan = proj._row_launches
    x = torch.zeros(2, 512, 1024)
    (only,) = plan(x)
    assert only[0] == slice(None) and only[2] == 1024
    trimmed = x[:, :328]
    launches = plan(trimmed)
    assert len(launches) == 2 and all(rs == 1024 for _, _, rs in launches)
    for b, (sl, rows, _) in enumerate(launches):
        assert sl == slice(b, b + 1) and rows.shape == (1, 328, 1024)
        assert rows.data_ptr() == trimmed[b].data_ptr()
    (one,) = plan(x[:1, :100])  # B == 1: the batch stride addresses nothing
    assert one[2] == 1024
    wide = torch.zeros(3, 40, 1536)[:, :, 256:1280]  # strided rows, uniform
    (w1,) = plan(wide)
    assert w1[2] == 1536
    col = torch.zeros(4, 1, 256)  # S == 1: rows at the batch stride
    (c1,) = plan(col)
    assert c1[2] == 256


def test_oracle_inputs_are_seeded_and_bf16_exact():
    a = ref.prologue_inputs(1, 1024, 2, seed=1001)
    b = ref.prologue_inputs(1, 1024, 2, seed=1001)
    assert all(torch.equal(a[k], b[k]) for k in a)
    assert torch.equal(a["qkv"], a["qkv"].to(torch.bfloat16).float())
    assert a["cos"].shape == (1024, 64)


def test_bench_rejects_more_than_one_gpu():
    proc = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"],
                          capture_output=True, text=True, timeout=300)
    assert proc.returncode == 2
    assert "one GPU" in proc.stderr


def test_package_loads_once():
    assert __graft_entry__.load_package() is __graft_entry__.load_package()


def test_negative_or_huge_sequence_strides_are_rejected(pkg, lib):
    """The tile DMA addresses K/V (forward) and Q/dO/K/V (backward) rows by a
    32-bit unsigned per-lane offset from a scalar row base, so a negative or
    >= 2^24 token stride must fail validation, before anything touches the device
    (the pointers below are never dereferenced)."""
    L = pkg._lib
    fake = 1 << 20  # 16-byte aligned, never read
    base = (1 << 15, 2048, 128)  # [B, S, H, 128] strides, elements
    a = L.AttnFwdArgs()
    a.q = a.k = a.v = a.out = fake
    a.B, a.Sq, a.Sk, a.H, a.hd, a.dtype, a.softmax_scale = 1, 64, 64, 16, 128, 0, 0.088
    for name in ("q_stride", "k_stride", "v_stride", "out_stride"):
        setattr(a, name, L.c_strides(base))
    for bad in (-2048, 1 << 24):
        a.k_stride = L.c_strides((1 << 15, bad, 128))
        assert lib.aa_attn_fwd(ctypes.byref(a), None) == L.AA_EUNSUPPORTED
        assert "sequence stride" in lib.aa_last_error().decode()
    b = L.AttnBwdArgs()
    b.dout = b.q = b.k = b.v = b.out = b.lse = b.dq = b.dk = b.dv = fake
    b.B, b.Sq, b.Sk, b.H, b.hd, b.dtype, b.softmax_scale = 1, 64, 64, 16, 128, 0, 0.088
    for name in ("dout_stride", "q_stride", "k_stride", "v_stride", "out_stride", "dq_stride",
                 "dk_stride", "dv_stride"):
        setattr(b, name, L.c_strides(base))
    for name in ("dout_stride", "q_stride", "k_stride", "v_stride"):
        setattr(b, name, L.c_strides((1 << 15, -2048, 128)))
        assert lib.aa_attn_bwd(ctypes.byref(b), None, 0, None) == L.AA_EUNSUPPORTED, name
        assert "sequence stride" in lib.aa_last_error().decode()
        setattr(b, name, L.c_strides(base))
