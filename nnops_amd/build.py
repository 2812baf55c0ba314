"""Build libnnops_amd.so (HIP kernels for gfx950 + the C++ front end) in-tree.

    python -m nnops_amd.build        # or nnops_amd.build.build()
    python -m nnops_amd.build --incremental   # only what changed

Each translation unit is compiled by hipcc for --offload-arch=gfx950 only,
objects go to nnops_amd/_build/, the shared library to nnops_amd/. Kernel TUs
are compiled with -ffp-contract=off (the int8 requant and the GELU epilogue
must round every float operation on its own to match the CPU bit for bit) and
without packed-FP32 instruction selection.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
BUILD = os.path.join(PKG, "_build")
LIB = os.path.join(PKG, "libnnops_amd.so")
# measurement probes (include/nnops_amd_diag.h), kept out of the product library
DIAG_SOURCES = ["csrc/kernels/diag.hip"]
DIAG_LIB = os.path.join(PKG, "libnnops_amd_diag.so")

SOURCES = [
    "csrc/kernels/gemm_i8.hip",
    "csrc/kernels/gemm_i8_noalloc.hip",
    "csrc/kernels/q4_1.hip",
    "csrc/kernels/q4_1_codec.hip",
    "csrc/kernels/quant.hip",
    "csrc/kernels/fp_out.hip",
    "csrc/kernels/fp_gemm.hip",
    "csrc/host/ops.cpp",
    "csrc/host/quant_linear.cpp",
    "csrc/host/capi_ops.cpp",
]

ARCH = "gfx950"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm install expected under /opt/rocm)")


def _flags(src: str) -> list[str]:
    common = [
        "-std=c++23", "-O3", "-fPIC", f"--offload-arch={ARCH}",
        "-I", os.path.join(ROOT, "include"),
        "-I", os.path.join(PKG, "include"),
        "-Wall", "-Wno-unused-function",
    ]
    if src.endswith(".hip"):
        common += [
            "-ffp-contract=off", "-fno-gpu-flush-denormals-to-zero",
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        ]
    else:
        common += ["-x", "hip"]  # host C++ that calls the HIP runtime
    return common


def _compile(src: str) -> str:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    cmd = [hipcc()] + _flags(src) + ["-c", os.path.join(PKG, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compile failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return obj


def _headers_mtime() -> float:
    t = 0.0
    for d in (os.path.join(ROOT, "include"), os.path.join(PKG, "include"), os.path.join(PKG, "csrc")):
        for root, _, files in os.walk(d):
            for f in files:
                if f.endswith((".h", ".hpp")):
                    t = max(t, os.path.getmtime(os.path.join(root, f)))
    return t


def _stale(src: str, hdr: float) -> bool:
    obj = os.path.join(BUILD, os.path.basename(src) + ".o")
    if not os.path.exists(obj):
        return True
    return os.path.getmtime(obj) < max(hdr, os.path.getmtime(os.path.join(PKG, src)))


def build(verbose: bool = False, incremental: bool = False) -> str:
    """Compile the sources and link the shared library; returns its path.
    Every source is compiled unless ``incremental`` (then only those older
    than their source or any header)."""
    os.makedirs(BUILD, exist_ok=True)
    hdr = _headers_mtime()
    todo = [s for s in SOURCES + DIAG_SOURCES if not incremental or _stale(s, hdr)]
    with cf.ThreadPoolExecutor(max_workers=max(1, min(8, len(todo)))) as ex:
        list(ex.map(_compile, todo))
    for srcs, lib in ((SOURCES, LIB), (DIAG_SOURCES, DIAG_LIB)):
        objs = [os.path.join(BUILD, os.path.basename(s) + ".o") for s in srcs]
        tmp = lib + ".tmp"
        cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", "-o", tmp] + objs
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            raise RuntimeError(f"link failed: {' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
        os.replace(tmp, lib)
        if verbose:
            print(f"built {lib}")
    return LIB


if __name__ == "__main__":
    build(verbose="-q" not in sys.argv, incremental="--incremental" in sys.argv)
