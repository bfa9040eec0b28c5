"""Builds the kf-hip C-ABI library for gfx950: kungfu_amd/lib/libkf_hip.so.

The library is compiled in-tree with hipcc (no JIT cache), so the built .so travels with the repository snapshot to
the GPU box. Every HIP translation unit is compiled with packed-FP32 instructions disabled.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
CSRC = os.path.join(HERE, "csrc")
OUT_DIR = os.path.join(HERE, "lib")
LIB = os.path.join(OUT_DIR, "libkf_hip.so")
OBJ_DIR = os.path.join(HERE, "build", "obj")

ARCH = "gfx950"
DEVICE_SOURCES = ["quant_act.hip", "gemv.hip", "gemv_k.hip", "gemm.hip", "gemm_q4k.hip", "gemm_kq.hip", "rows.hip", "rows_mma.hip", "noalloc.hip", "probe.hip"]
HOST_SOURCES = ["api.cpp", "host_quant.cpp", "gguf.cpp", "knobs.cpp"]

COMMON = ["-O3", "-fPIC", "-std=c++17", "-Wall", "-I" + os.path.join(ROOT, "include"), "-I" + CSRC]
DEVICE_FLAGS = [f"--offload-arch={ARCH}", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-ffp-contract=fast-honor-pragmas"]
# per-source additions: the int8 GEMMs take the matrix-core results in ordinary vector registers (no copies out of
# the accumulation registers before the float rescale that follows every MFMA)
SOURCE_FLAGS = {"gemm.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"]}


def hipcc() -> str:
    p = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(p):
        raise RuntimeError("hipcc not found (ROCm toolchain required to build kf-hip)")
    return p


def _compile(src: str, obj: str, device: bool) -> None:
    cmd = [hipcc(), "-c", src, "-o", obj] + COMMON
    cmd += (["-x", "hip"] + DEVICE_FLAGS + SOURCE_FLAGS.get(os.path.basename(src), [])) if device else ["-D__HIP_PLATFORM_AMD__"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")


def build(verbose: bool = False) -> str:
    """Compiles every source and links the shared library; returns its path."""
    os.makedirs(OBJ_DIR, exist_ok=True)
    os.makedirs(OUT_DIR, exist_ok=True)
    jobs = [(os.path.join(CSRC, s), os.path.join(OBJ_DIR, s + ".o"), True) for s in DEVICE_SOURCES]
    jobs += [(os.path.join(CSRC, s), os.path.join(OBJ_DIR, s + ".o"), False) for s in HOST_SOURCES]
    workers = min(len(jobs), max(1, min(8, os.cpu_count() or 1)))
    with cf.ThreadPoolExecutor(workers) as ex:
        futs = [ex.submit(_compile, *j) for j in jobs]
        for f in futs:
            f.result()
    tmp = LIB + ".tmp"
    cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", "-o", tmp] + [j[1] for j in jobs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print("built", LIB)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
