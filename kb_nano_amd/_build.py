"""Builds ``libkbn_fp8.so`` (the gfx950 HIP kernels plus their C-ABI) in-tree.

``python -m kb_nano_amd._build`` or ``__graft_entry__.build()`` compiles every
``csrc/*.hip`` file with ``hipcc --offload-arch=gfx950`` and links one shared
library next to this file.  The library is loaded with ctypes by
``kb_nano_amd._lib``; nothing is JIT-compiled at run time.
"""
from __future__ import annotations

import concurrent.futures as cf
import glob
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB_NAME = "libkbn_fp8.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)
OBJ_DIR = os.path.join(HERE, "_build")
ARCH = os.environ.get("KBN_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    # packed fp32 VALU ops stay off: the kernels are written for scalar fp32
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-command-line-argument",
]


def _hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; the ROCm toolchain is required to build kb_nano_amd")
    return path


def _generate_silu_lut() -> None:
    """Compile and run gen_silu_lut.cpp (host code) to write the bf16 SiLU
    table that quant.hip includes."""
    cxx = shutil.which("g++") or shutil.which("c++")
    if cxx is None:
        raise RuntimeError("a host C++ compiler (g++) is needed to generate the SiLU table")
    gen = os.path.join(OBJ_DIR, "gen_silu_lut")
    src = os.path.join(CSRC, "gen_silu_lut.cpp")
    r = subprocess.run([cxx, "-O2", "-std=c++17", "-o", gen, src], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"building {src} failed:\n{r.stderr}")
    r = subprocess.run([gen, os.path.join(OBJ_DIR, "silu_lut.inc")], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"gen_silu_lut failed:\n{r.stderr}")


# Per-file options.  gemm.hip's tiles keep their MFMA accumulators in VGPRs
# (the FP32 scale contract's per-block rescale is then one multiply per
# element, not an AGPR read, multiply and write: grouped cfg4 GEMMs with a
# checkpoint's fp32 weight scales 15-17% faster); gemm_big.hip's 256x256
# tiles need the AGPRs for their 256 accumulators per lane and stay without.
FILE_FLAGS = {
    "gemm.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=true"],
}


def _compile(src: str, hipcc: str) -> str:
    obj = os.path.join(OBJ_DIR, os.path.basename(src) + ".o")
    extra = FILE_FLAGS.get(os.path.basename(src), [])
    cmd = [hipcc, *HIPCC_FLAGS, *extra, "-I", CSRC, "-I", OBJ_DIR, "-c", src, "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    return obj


BENCH_CSRC = os.path.join(HERE, "bench_csrc")
BENCH_LIB_PATH = os.path.join(HERE, "libkbn_bench.so")


def build_bench(hipcc: str | None = None) -> str:
    """Compile ``bench_csrc/*.hip`` (bench.py's streaming probes, not part of
    the operator library) into ``libkbn_bench.so``; returns its path."""
    hipcc = hipcc or _hipcc()
    os.makedirs(OBJ_DIR, exist_ok=True)
    sources = sorted(glob.glob(os.path.join(BENCH_CSRC, "*.hip")))
    objs = [_compile(s, hipcc) for s in sources]
    tmp = BENCH_LIB_PATH + ".tmp"
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, BENCH_LIB_PATH)
    return BENCH_LIB_PATH


def build(verbose: bool = False) -> str:
    """Compile all HIP sources and link ``libkbn_fp8.so`` (and bench.py's
    ``libkbn_bench.so``); returns the operator library's path."""
    hipcc = _hipcc()
    os.makedirs(OBJ_DIR, exist_ok=True)
    _generate_silu_lut()
    sources = sorted(glob.glob(os.path.join(CSRC, "*.hip")))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    with cf.ThreadPoolExecutor(max_workers=min(8, len(sources))) as ex:
        objs = list(ex.map(lambda s: _compile(s, hipcc), sources))
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{' '.join(cmd)}\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB_PATH)
    build_bench(hipcc)
    if verbose:
        print(f"built {LIB_PATH} from {len(sources)} sources, and {BENCH_LIB_PATH}", file=sys.stderr)
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
