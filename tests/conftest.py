"""Shared fixtures: the package under test, the CPU oracle, parity checks.

GPU tests are marked `gpu` and skip when no GPU is visible; everything else
runs on the CPU.
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

import __graft_entry__  # noqa: E402

MAX_ABS = 2e-2
REL_L2 = 5e-3


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def pytest_collection_modifyitems(config, items):
    if torch.cuda.is_available():
        return
    skip = pytest.mark.skip(reason="no GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


@pytest.fixture(scope="session")
def pkg():
    return __graft_entry__.load_package()


@pytest.fixture(scope="session")
def fp8(pkg):
    """The opt-in rowquant module (anima_flat_amd.kernels.fp8)."""
    import importlib

    return importlib.import_module("anima_flat_amd.kernels.fp8")


@pytest.fixture(scope="session")
def proj(pkg):
    """The opt-in fused-projection module (anima_flat_amd.kernels.proj)."""
    import importlib

    return importlib.import_module("anima_flat_amd.kernels.proj")


@pytest.fixture(scope="session")
def dev():
    return torch.device("cuda:0")


def parity(actual, expected, max_abs=MAX_ABS, rel_l2=REL_L2, name=""):
    """max |a - e| <= max_abs and ||a - e|| / ||e|| <= rel_l2 (fp32 on the CPU)."""
    a = actual.detach().float().cpu()
    e = expected.detach().float().cpu()
    assert a.shape == e.shape, f"{name}: shape {tuple(a.shape)} != {tuple(e.shape)}"
    assert torch.isfinite(a).all(), f"{name}: non-finite values"
    if a.numel() == 0:
        return 0.0, 0.0
    err = a - e
    mx = err.abs().max().item()
    rl = (err.norm() / e.norm().clamp_min(1e-30)).item()
    print(f"[parity] {name}: max_abs={mx:.3e} rel_l2={rl:.3e}", flush=True)
    assert mx <= max_abs, f"{name}: max_abs {mx:.3e} > {max_abs}"
    assert rl <= rel_l2, f"{name}: rel_l2 {rl:.3e} > {rel_l2}"
    return mx, rl
