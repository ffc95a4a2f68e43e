"""Builds libanima_attn.so from csrc/*.hip with hipcc for gfx950.

Objects go to `_build/` next to this file and the library to
`libanima_attn.so` in this directory, where `_lib.py` loads it from. Every
source compiles in parallel; nothing is cached between calls (the caller asks
for a build, so it gets one).

Run as a script to build: ``python anima-flat_amd/build.py``.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

HERE = Path(__file__).resolve().parent
CSRC = HERE / "csrc"
BUILD = HERE / "_build"
LIB_NAME = "libanima_attn.so"
LIB_PATH = HERE / LIB_NAME
SOURCES = (
    "abi.hip", "prologue.hip", "ctx_scale.hip", "context.hip", "rowquant.hip", "attn_fwd.hip",
    "attn_fwd_pp.hip", "attn_fwd_d384.hip", "attn_bwd.hip", "attn_bwd_dkdv.hip", "qkv_proj.hip",
)
ARCH = "gfx950"
# The measurement's MFMA-rate calibration (bench.py), a library of its own so
# that the attention library holds only the path's entry points.
CALIB_SOURCE = "calib_mfma.hip"
CALIB_LIB_PATH = HERE / "libanima_calib.so"

# Packed fp32 VALU forms are disabled for all device code: the compiler then
# emits only scalar v_fma_f32/v_mul_f32 for float arithmetic.
DEVICE_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


RESOURCE_REMARK = "-Rpass-analysis=kernel-resource-usage"

# Per-source extra flags. attn_fwd.hip and attn_bwd_dkdv.hip run one wave per
# SIMD, where the compiler would otherwise give every MFMA accumulator the
# AGPR file; their score accumulators must be VGPRs (the VALU reads them), so
# the builtin MFMAs are compiled in the VGPR form and the output accumulators
# are pinned to AGPRs through inline asm.
SOURCE_FLAGS: dict[str, list[str]] = {
    "attn_fwd.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
    "attn_bwd_dkdv.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
}


def hipcc() -> str:
    """Path of hipcc (ROCM_PATH/bin, then PATH)."""
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = Path(rocm) / "bin" / "hipcc"
    if cand.exists():
        return str(cand)
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found: set ROCM_PATH or put hipcc on PATH")
    return found


SGPR_SPILL_WARNINGS: list[str] = []


def _check_resources(stderr: str, src: str) -> None:
    """Fails the build if any kernel of `src` uses scratch memory or spills VGPRs,
    and records (and prints) every kernel that spills SGPRs.

    The remarks come from -Rpass-analysis=kernel-resource-usage. Every kernel
    here is written to keep its working set in registers and LDS; a VGPR spill
    means an unroll or an indexing pattern went wrong, and costs an order of
    magnitude in speed, so it is treated as a build error. SGPR spills go to
    VGPR lanes (v_writelane / v_readlane, no memory); they cost a few
    instructions where they occur, so they are reported, not rejected."""
    name = None
    for line in stderr.splitlines():
        if "remark:" not in line:
            continue
        body = line.split("remark:", 1)[1].strip()
        if body.startswith("Function Name:"):
            name = body.split(":", 1)[1].split("[")[0].strip()
        elif body.startswith("ScratchSize [bytes/lane]:") or body.startswith("VGPRs Spill:"):
            value = int(body.split(":", 1)[1].split("[")[0])
            if value != 0:
                raise RuntimeError(f"{src}: kernel {name}: {body.split('[-R')[0].strip()}")
        elif body.startswith("SGPRs Spill:"):
            value = int(body.split(":", 1)[1].split("[")[0])
            if value != 0:
                msg = f"{src}: kernel {name}: {value} SGPRs spilled to VGPR lanes"
                SGPR_SPILL_WARNINGS.append(msg)
                print(f"warning: {msg}", file=sys.stderr, flush=True)


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        # hipcc's host pass warns about the packed-fp32 feature; keep real errors.
        err = "\n".join(
            line for line in proc.stderr.splitlines() if "packed-fp32-ops" not in line
        )
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{err}")
    if RESOURCE_REMARK in cmd:
        _check_resources(proc.stderr, cmd[cmd.index("-c") + 1])


def build(verbose: bool = False) -> Path:
    """Compile every source, link libanima_attn.so and the calibration library
    libanima_calib.so; returns the attention library's path."""
    cc = hipcc()
    SGPR_SPILL_WARNINGS.clear()
    BUILD.mkdir(exist_ok=True)
    objs = []
    cmds = []
    for src in SOURCES + (CALIB_SOURCE,):
        obj = BUILD / (Path(src).stem + ".o")
        if src != CALIB_SOURCE:
            objs.append(str(obj))
        cmds.append([cc, *DEVICE_FLAGS, *SOURCE_FLAGS.get(src, []), RESOURCE_REMARK, "-c",
                     str(CSRC / src), "-o", str(obj)])
    workers = max(1, min(len(cmds), os.cpu_count() or 1, 8))
    with ThreadPoolExecutor(workers) as pool:
        for cmd, _ in zip(cmds, pool.map(_run, cmds)):
            if verbose:
                print(" ".join(cmd), flush=True)
    tmp = LIB_PATH.with_suffix(".so.tmp")
    link = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *objs]
    if verbose:
        print(" ".join(link), flush=True)
    _run(link)
    os.replace(tmp, LIB_PATH)
    ctmp = CALIB_LIB_PATH.with_suffix(".so.tmp")
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(ctmp),
          str(BUILD / (Path(CALIB_SOURCE).stem + ".o"))])
    os.replace(ctmp, CALIB_LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
