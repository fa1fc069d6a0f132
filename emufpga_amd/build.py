"""Build libemuhip.so (hand-written gfx950 HIP kernels + C ABI) in-tree.

Run as ``python -m emufpga_amd.build``.  The library is compiled with hipcc for
gfx950 only; packed FP32 instructions are disabled for every device pass.
"""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIB = PKG / "libemuhip.so"
ARCH = os.environ.get("EMU_OFFLOAD_ARCH", "gfx950")

SOURCES = ["core.hip", "qmv.hip", "limb.hip", "mfma.hip", "ops.hip", "attn.hip", "moe.hip", "model.hip", "files.hip"]

FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    "-Wno-unused-parameter",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = Path(rocm) / "bin" / "hipcc"
    return str(cand) if cand.exists() else "hipcc"


def build(verbose: bool = False) -> Path:
    """Compile every source into ``emufpga_amd/libemuhip.so`` (always rebuilds)."""
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), *FLAGS, "-o", str(tmp), *[str(CSRC / s) for s in SOURCES]]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed ({res.returncode}) building {LIB.name}")
    # Warnings about the packed-fp32 feature come from the host pass and are harmless.
    noise = [ln for ln in res.stderr.splitlines() if ln.strip() and "packed-fp32-ops" not in ln]
    if verbose and noise:
        sys.stderr.write("\n".join(noise) + "\n")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
