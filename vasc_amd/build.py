"""Builds ``vasc_amd/libvasc_hip.so`` from ``vasc_amd/csrc`` with hipcc for gfx950.

Usage: ``python -m vasc_amd.build`` (also called by ``__graft_entry__.build``).
Objects go to ``vasc_amd/_build/``; the shared library sits next to this
file so it travels with the source tree.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libvasc_hip.so"
ARCH = os.environ.get("VASC_OFFLOAD_ARCH", "gfx950")

COMMON_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    # Packed FP32 VALU ops are disabled: hipcc must not form v_pk_*_f32.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-command-line-argument",
]

# Per-source extra flags. The selection and innovation arithmetic must round
# every float32 operation separately to stay bit-identical with the oracle.
SOURCES = {
    "capi.cpp": [],
    # MFMA accumulators in VGPRs (no AGPR round trips in the softmax loop);
    # no NaN canonicalisation around the running max.
    "attn.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form", "-fno-honor-nans"],
    "pack.hip": [],
    # products and sums round separately except where the code fuses them
    # explicitly (fmaf in the LayerNorm and rotary of transform_row)
    "layout.hip": ["-ffp-contract=off"],
    "pool.hip": ["-ffp-contract=off"],
    "select.hip": ["-ffp-contract=off", "-Wshadow"],
    # the residual products and sums round separately, as torch's bf16 ops do
    "block.hip": ["-ffp-contract=off"],
}


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found (ROCm is required to build libvasc_hip.so)")
    return path


def _compile(src: str, extra: list[str]) -> Path:
    obj = BUILD / (Path(src).stem + ".o")
    cmd = [hipcc(), "-x", "hip", "-c", str(CSRC / src), "-o", str(obj), *COMMON_FLAGS, *extra]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    return obj


def build(verbose: bool = True) -> Path:
    """Compile every source and link the shared library. Returns its path."""
    BUILD.mkdir(exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 4)) as pool:
        objs = list(pool.map(lambda kv: _compile(*kv), SOURCES.items()))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} ({LIB.stat().st_size} bytes, arch {ARCH})")
    return LIB


if __name__ == "__main__":
    build()
    sys.exit(0)
