"""Build libvolundr_sampling.so (the C-ABI HIP library) in-tree with hipcc for gfx950.

    python volundr-mlx_amd/volundr_amd/build.py        # or volundr_amd.build.build()

The library lands next to this file, so it travels with the source tree; nothing is installed.
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG.parent / "csrc"
LIB = PKG / "libvolundr_sampling.so"
OBJ = PKG.parent / "_build"
SOURCES = ["vs_api.hip", "vs_sample.hip", "vs_verify.hip", "vs_draft.hip", "vs_lmhead.hip"]
ARCH = os.environ.get("VS_OFFLOAD_ARCH", "gfx950")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-ffp-contract=off",                       # no a*b+c -> fma: the sampler's fp32 arithmetic must match NumPy
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _compile(src: str, extra=()) -> Path:
    out = OBJ / (Path(src).stem + ("_dev" if extra else "") + ".o")
    cmd = [HIPCC, *FLAGS, *extra, "-c", str(CSRC / src), "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stderr}")
    return out


def build(verbose: bool = False, out: Path = LIB, defines=()) -> Path:
    """Compile every HIP source and link the shared library. Always rebuilds. `defines` (e.g. ["VS_TRACE"])
    make a development variant, which should be written somewhere other than the shipped path."""
    OBJ.mkdir(exist_ok=True)
    extra = tuple(f"-D{d}" for d in defines)
    with ThreadPoolExecutor(max_workers=len(SOURCES)) as ex:
        objs = list(ex.map(lambda s: _compile(s, extra), SOURCES))
    LIB_ = Path(out)
    tmp = LIB_.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stderr}")
    os.replace(tmp, LIB_)
    if verbose:
        print(f"built {LIB_}")
    return LIB_


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
