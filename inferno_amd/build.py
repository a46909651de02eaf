"""Build the gfx950 launch layer (libinferno_hip.so) in-tree with hipcc.

Usage: ``python -m inferno_amd.build`` (or ``__graft_entry__.build()``).
Object files go to ``_build/`` at the repository root; the shared library is
written next to this file so it travels with the source tree.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = ROOT / "_build"
LIB = PKG / "libinferno_hip.so"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# -packed-fp32-ops: hipcc must not form v_pk_{add,mul,fma}_f32 from scalar fp32 code.
COMMON = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics",
    "-Wno-unused-result",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
]

SOURCES = ["capi.cpp", "attn_fwd.hip", "attn_bwd.hip", "decode.hip", "softmax.hip"]


def _compile(src: Path, obj: Path) -> None:
    cmd = [HIPCC, *COMMON, "-x", "hip", "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")


def build(verbose: bool = True) -> Path:
    BUILD.mkdir(exist_ok=True)
    objs = []
    jobs = []
    with cf.ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        for s in SOURCES:
            src = CSRC / s
            obj = BUILD / (s.replace(".", "_") + ".o")
            objs.append(obj)
            jobs.append(ex.submit(_compile, src, obj))
        for j in jobs:
            j.result()
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}", file=sys.stderr)
    return LIB


if __name__ == "__main__":
    build()
