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

SOURCES = ["capi.cpp", "attn_fwd.hip", "attn_fwd_bf16.hip", "attn_bwd.hip", "attn_bwd_bf16.hip", "decode.hip", "softmax.hip", "elementwise.hip", "nn.hip",
           "capi_nn.cpp", "gemm.cpp"]


def _compile(src: Path, obj: Path) -> None:
    cmd = [HIPCC, *COMMON, "-x", "hip", "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")


# The C++ Tensor / autograd layer (host code only; g++ with the HIP runtime API headers).
HOST_LIB = PKG / "libinferno.so"
CPP = PKG / "cpp"
CPP_SOURCES = ["dtype.cpp", "storage.cpp", "hipctx.cpp", "tensor.cpp", "engine.cpp", "softmax.cpp", "attention.cpp", "mask_ops.cpp",
               "nn_ops.cpp", "modules.cpp", "checkpoint.cpp"]
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
CXX = os.environ.get("CXX", "g++")
# -ffp-contract=off: the CPU-device branches keep the reference's separate
# product and sum roundings.
HOST_FLAGS = ["-std=c++20", "-O2", "-fPIC", "-ffp-contract=off", "-Wall", "-Wno-unused-function",
              "-D__HIP_PLATFORM_AMD__", f"-I{ROOT / 'include'}", f"-I{ROCM / 'include'}"]
DRIVER_SRC = ROOT / "tests" / "cpp" / "api_driver.cpp"
APP_SRC = PKG / "app" / "gpt.cpp"
APP = PKG / "gpt"
DRIVER = ROOT / "tests" / "cpp" / "api_driver"


def _run(cmd, what):
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"{what} failed:\n{' '.join(map(str, cmd))}\n{r.stdout}\n{r.stderr}")


def build_host(verbose: bool = True) -> Path:
    """libinferno.so (Tensor, autograd, ops) linked against libinferno_hip.so, plus the test driver."""
    BUILD.mkdir(exist_ok=True)
    objs = []
    with cf.ThreadPoolExecutor(max_workers=min(8, len(CPP_SOURCES))) as ex:
        jobs = []
        for src in CPP_SOURCES:
            obj = BUILD / ("host_" + src.replace(".", "_") + ".o")
            objs.append(obj)
            jobs.append(ex.submit(_run, [CXX, *HOST_FLAGS, "-c", str(CPP / src), "-o", str(obj)], f"g++ {src}"))
        for j in jobs:
            j.result()
    tmp = HOST_LIB.with_suffix(".so.tmp")
    _run([CXX, "-shared", "-o", str(tmp), *map(str, objs), f"-L{PKG}", "-linferno_hip", f"-L{ROCM / 'lib'}",
          "-lamdhip64", "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{ROCM / 'lib'}"], "link libinferno.so")
    os.replace(tmp, HOST_LIB)
    if DRIVER_SRC.exists():
        _run([CXX, *HOST_FLAGS, str(DRIVER_SRC), "-o", str(DRIVER), f"-L{PKG}", "-linferno", "-linferno_hip",
              f"-L{ROCM / 'lib'}", "-lamdhip64", f"-Wl,-rpath,{PKG}", f"-Wl,-rpath,{ROCM / 'lib'}",
              "-Wl,-rpath,$ORIGIN/../../inferno_amd"], "build api_driver")
    _run([CXX, *HOST_FLAGS, str(APP_SRC), "-o", str(APP), f"-L{PKG}", "-linferno", "-linferno_hip",
          f"-L{ROCM / 'lib'}", "-lamdhip64", "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{ROCM / 'lib'}"], "build gpt app")
    if verbose:
        print(f"built {HOST_LIB}", file=sys.stderr)
    return HOST_LIB


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
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs),
           f"-L{ROCM / 'lib'}", "-lhipblaslt", f"-Wl,-rpath,{ROCM / 'lib'}"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}", file=sys.stderr)
    build_host(verbose)
    return LIB


if __name__ == "__main__":
    build()
