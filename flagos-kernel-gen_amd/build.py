"""Build libmw4a8.so (HIP kernels + C ABI) for gfx950 with hipcc.

Usage: ``python flagos-kernel-gen_amd/build.py`` (or ``__graft_entry__.build()``).
Objects go to ``flagos-kernel-gen_amd/_build/``; the shared library is
written next to this file. Every call recompiles.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
OBJ_DIR = os.path.join(HERE, "_build")
LIB_NAME = "libmw4a8.so"
LIB_PATH = os.path.join(HERE, LIB_NAME)
ARCH = "gfx950"

# the grouped GEMM's kernel template (gemm_kernel.h) is instantiated per row
# source in the gemm_*.hip files, which compile in parallel
SOURCES = ("gemm_routed.hip", "gemm_csr.hip", "gemm_repacked.hip", "gemm_debug_routed.hip", "gemm_debug_csr.hip",
           "gemm_debug_repacked.hip", "api.hip", "moe_align.hip", "grouped_gemm.hip", "moe_layer.hip",
           "measure.hip")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # no packed-fp32 VALU instructions in device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found; the HIP toolchain is required to build libmw4a8.so")


# The debug exports' extra stores make their fully unrolled loops larger than
# the unroller's default limit for unroll pragmas; a higher limit keeps their
# loop structure that of the product kernels.
EXTRA_FLAGS = {src: ["-mllvm", "-pragma-unroll-threshold=200000"]
               for src in ("gemm_debug_routed.hip", "gemm_debug_csr.hip", "gemm_debug_repacked.hip")}


def resources_path(src: str) -> str:
    """Per-kernel register / scratch / occupancy report of one source
    (the compiler's kernel-resource-usage remarks, written by every build)."""
    return os.path.join(OBJ_DIR, os.path.splitext(src)[0] + ".resources.txt")


def _compile(src: str) -> str:
    obj = os.path.join(OBJ_DIR, os.path.splitext(src)[0] + ".o")
    cmd = [hipcc(), "-x", "hip", *HIPCC_FLAGS, *EXTRA_FLAGS.get(src, []), "-Rpass-analysis=kernel-resource-usage",
           "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
    remarks, noise, in_remark = [], [], False
    for ln in r.stderr.splitlines():
        if "kernel-resource-usage" in ln:
            remarks.append(ln)
            in_remark = True
        elif in_remark and (ln.lstrip().startswith("|") or ln.lstrip().split("|")[0].strip().isdigit()):
            continue   # the source snippet printed under a remark
        else:
            in_remark = False
            if "packed-fp32-ops" not in ln and ln.strip() and not ln.startswith("In file included from"):
                noise.append(ln)
    with open(resources_path(src), "w") as f:
        f.write("\n".join(remarks) + "\n")
    if noise:
        sys.stderr.write(f"[build] {src}:\n" + "\n".join(noise) + "\n")
    return obj


def build(verbose: bool = True) -> str:
    os.makedirs(OBJ_DIR, exist_ok=True)
    with ThreadPoolExecutor(max_workers=max(1, min(len(SOURCES), os.cpu_count() or 1))) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", tmp, *objs]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"[build] {LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build()
