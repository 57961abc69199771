"""Build the gfx950 HIP library ``libinferrous_w8a8.so`` in-tree.

Every HIP source is compiled by hipcc for gfx950 only, with
``-ffp-contract=off`` (no FMA contraction: the epilogue's two RN multiplies
and the residual's RN add must stay separate operations) and packed-FP32
instructions disabled (``-Xclang -target-feature -Xclang -packed-fp32-ops``).
Objects go to ``inferrous_amd/_build/``; the shared library next to this file.

Usage: ``python -m inferrous_amd.build`` (or ``build()`` from Python).
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
OBJ = PKG / "_build"
LIB = PKG / "libinferrous_w8a8.so"
SOURCES = ["abi.hip", "quantize.hip", "gemv.hip", "gemm.hip", "head.hip", "synth.hip", "sequence.hip"]
ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: cannot build the gfx950 library")


def compile_flags() -> list[str]:
    return [f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-ffp-contract=off",
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
            "-mllvm", "-amdgpu-kernarg-preload-count=16",
            "-Wall", "-Wno-unused-function", "-I", str(PKG.parent / "include")]


def build(verbose: bool = False) -> Path:
    cc = hipcc()
    OBJ.mkdir(exist_ok=True)

    def one(src: str) -> Path:
        obj = OBJ / (src + ".o")
        cmd = [cc, *compile_flags(), "-c", str(CSRC / src), "-o", str(obj)]
        r = subprocess.run(cmd, capture_output=True, text=True)
        noise = "is not a recognized feature for this target"
        err = "\n".join(l for l in (r.stderr or "").splitlines() if noise not in l)
        if r.returncode != 0:
            lines = [l for l in err.splitlines() if "error" in l][:20]
            raise RuntimeError(f"hipcc failed for {src}:\n" + "\n".join(lines))
        if verbose and err.strip():
            print(err, file=sys.stderr)
        return obj

    with ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 1)) as ex:
        objs = list(ex.map(one, SOURCES))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose=True))
