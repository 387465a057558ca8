"""Build libkomp_hip.so, the gfx950 HIP library behind the C ABI of include/komp_abi.h.

    python -m comp_amd.build            # compile every HIP source and link comp_amd/libkomp_hip.so

Each source compiles to an object in comp_amd/_build/ (in parallel), then hipcc links the shared library in-tree, next
to this file, where comp_amd._abi loads it.  Flags: gfx950 only, -O3, no fast-math (the quantizers need correctly
rounded f32 division), packed-FP32 instructions disabled.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libkomp_hip.so")
SOURCES = ("abi.hip", "quant.hip", "gemv.hip", "gemv_fused.hip", "gemv_more.hip", "gemv_more_fused.hip",
           "gemv_q4_k.hip", "gemv_q4_k_fused.hip", "gemv_tq2.hip", "gemv_tq2_bytes.hip", "gemv_tq2_stamp.hip", "gemv_tq2_mfma.hip", "gemv_q4.hip",
           "gemv_q4_bytes.hip", "gemv_q4k.hip", "gemv_q4k_fused.hip", "gemv_q8.hip", "gemv_q8_fused.hip", "gemm.hip", "split.hip")
ARCH = "gfx950"


def hipcc():
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found: the HIP library needs ROCm's hipcc")
    return path


def compile_flags():
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-Wall",
        "-Xclang",
        "-target-feature",
        "-Xclang",
        "-packed-fp32-ops",
        # the first 16 kernel-argument dwords arrive in SGPRs at wave launch (gfx950 kernarg preloading)
        "-mllvm",
        "-amdgpu-kernarg-preload-count=16",
        # MFMA results in ordinary VGPRs (the matrix-core GEMM converts every result right away; without this the
        # compiler parks them in AGPRs and copies each one back)
        "-mllvm",
        "-amdgpu-mfma-vgpr-form",
    ]


def _compile(src):
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc(), *compile_flags(), "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    errs = "\n".join(ln for ln in (r.stdout + r.stderr).splitlines() if "packed-fp32-ops" not in ln)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{errs}")
    return obj


def build(verbose=False):
    """Compile every HIP source for gfx950 and link comp_amd/libkomp_hip.so.  Returns the library path."""
    os.makedirs(BUILD, exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 1)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}{r.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}")
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
