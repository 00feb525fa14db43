"""Builds libsharpinference_hip.so for gfx950 with hipcc, in-tree.

    python -m sharpinference_amd.build

Every HIP source is compiled with packed-FP32 instruction selection turned
off (the compiler emits scalar v_fma_f32 / v_add_f32 instead of
v_pk_*_f32) and with floating-point contraction off, so every FMA in the
kernels is an explicit fmaf() and the block decoders round each operation
on its own.
"""
from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
CSRC = os.path.join(PKG, "csrc")
BUILD_DIR = os.path.join(PKG, "_build")
LIB_NAME = "libsharpinference_hip.so"
LIB_PATH = os.path.join(PKG, LIB_NAME)
HOST_DIR = os.path.join(PKG, "host")
HOST_LIB_PATH = os.path.join(PKG, "libsharpinference_hip_host.so")
ARCH = os.environ.get("SI_HIP_ARCH", "gfx950")

SOURCES = [
    "si_abi.cpp",
    "si_model.cpp",
    "si_gemv.hip",
    "si_prefill.hip",
    "si_decode.hip",
    "si_rwkv.hip",
    "si_rwkv_program.cpp",
    "si_gguf.cpp",
    "si_transformer.hip",
    "si_ops.cpp",
    "si_batch.hip",
    "si_batch_abi.cpp",
    "si_t0.hip",
    "si_t0_abi.cpp",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found: the HIP backend cannot be built")


def common_flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-ffp-contract=off",
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        # leading scalar kernel arguments arrive in SGPRs at wave launch
        # (gfx950 kernarg preload), so a kernel's first loads do not wait
        # for a kernel-argument fetch
        "-mllvm", "-amdgpu-kernarg-preload-count=16",
        "-Wall",
        "-Wno-unused-result",
        f"-I{os.path.join(ROOT, 'include')}",
        f"-I{CSRC}",
    ]


def _compile(src: str) -> str:
    obj = os.path.join(BUILD_DIR, os.path.basename(src) + ".o")
    cmd = [_hipcc(), *common_flags(), "-x", "hip", "-c", os.path.join(CSRC, src), "-o", obj]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # The host pass does not know the packed-fp32 feature name and says so;
    # drop exactly that line and surface everything else.
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in proc.stderr.splitlines() if noise not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{err}")
    if err.strip():
        sys.stderr.write(err + "\n")
    return obj


def build(verbose: bool = False) -> str:
    """Compile all sources and link the shared library; returns its path."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as pool:
        objs = list(pool.map(_compile, SOURCES))
    tmp = LIB_PATH + ".tmp"
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, LIB_PATH)
    build_host()
    if verbose:
        print(f"built {LIB_PATH}")
        print(f"built {HOST_LIB_PATH}")
    return LIB_PATH


def build_host() -> str:
    """The C++ host interface (instruction contract, registry, VM executor)
    as libsharpinference_hip_host.so, linked against the HIP library in the
    same directory (found through an $ORIGIN run path)."""
    tmp = HOST_LIB_PATH + ".tmp"
    cmd = [os.environ.get("CXX", "g++"), "-O2", "-std=c++17", "-fPIC", "-shared", "-Wall", "-Wextra",
           f"-I{os.path.join(ROOT, 'include')}",
           *[os.path.join(HOST_DIR, f) for f in sorted(os.listdir(HOST_DIR)) if f.endswith(".cpp")],
           f"-L{PKG}", "-lsharpinference_hip", "-Wl,-rpath,$ORIGIN", "-o", tmp]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"host library build failed:\n{proc.stderr}")
    if proc.stderr.strip():
        sys.stderr.write(proc.stderr)
    os.replace(tmp, HOST_LIB_PATH)
    return HOST_LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
