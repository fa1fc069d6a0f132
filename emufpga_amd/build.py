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

SOURCES = ["core.hip", "qmv.hip", "limb.hip", "mfma.hip", "ops.hip", "attn.hip", "moe.hip", "model.hip", "files.hip",
           "cache.hip"]

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


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed ({res.returncode}): {' '.join(cmd[-3:])}")
    # Warnings about the packed-fp32 feature come from the host pass and are harmless.
    noise = [ln for ln in res.stderr.splitlines() if ln.strip() and "packed-fp32-ops" not in ln]
    if verbose and noise:
        sys.stderr.write("\n".join(noise) + "\n")


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every source into ``emufpga_amd/libemuhip.so`` (always rebuilds).

    Each source compiles to its own object in ``_build/`` in parallel, then
    one link makes the shared library."""
    from concurrent.futures import ThreadPoolExecutor

    objdir = PKG / "_build"
    objdir.mkdir(exist_ok=True)
    compile_flags = [f for f in FLAGS if f != "-shared"]
    objs = [objdir / (Path(s).stem + ".o") for s in SOURCES]
    cmds = [[hipcc(), *compile_flags, "-c", "-o", str(o), str(CSRC / s)] for s, o in zip(SOURCES, objs)]
    jobs = jobs or min(len(cmds), max(1, int(os.environ.get("MAX_JOBS", os.cpu_count() or 1))))
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        for fut in [pool.submit(_run, c, verbose) for c in cmds]:
            fut.result()
    tmp = LIB.with_suffix(".so.tmp")
    _run([hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", "-o", str(tmp), *[str(o) for o in objs]], verbose)
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
