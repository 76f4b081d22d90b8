"""Register, scratch and occupancy of every compiled kernel, from the
compiler's kernel-resource-usage report that each build writes next to its
objects (flagos-kernel-gen_amd/_build/*.resources.txt). No GPU needed.

Every product kernel must run without scratch (a spill turns register
traffic into memory traffic: spilling variants measured 3-4x slower) and
with at least two waves per SIMD. The debug-export kernels (template flag
DEBUGP, the `Lb1E` after the row-source mode in the mangled name) are only
run by the tests; their extra partial-sum stores may spill, which costs test
time only, so they are reported but not held to the bar."""

import glob
import os
import re

import pytest

from conftest import ROOT

PKG = os.path.join(ROOT, "flagos-kernel-gen_amd")
OBJ_DIR = os.path.join(PKG, "_build")


def _kernels():
    out = {}
    for path in sorted(glob.glob(os.path.join(OBJ_DIR, "*.resources.txt"))):
        name = None
        for line in open(path):
            m = re.search(r"Function Name: (\S+)", line)
            if m:
                name = m.group(1)
                out[name] = {"file": os.path.basename(path)}
                continue
            m = re.search(r"remark:\s+(VGPRs|AGPRs|ScratchSize \[bytes/lane\]|Occupancy \[waves/SIMD\]): (\d+)", line)
            if m and name:
                key = m.group(1).split()[0]
                out[name][key] = int(m.group(2))
    return out


def _is_debug(name):
    # w4a8_gemm_kernel<BM, WN, NW, GS, KCG, RD, ZSG, RMODE, DEBUGP, FAST, ZSV, WPE>
    m = re.match(r"_ZN5mw4a816w4a8_gemm_kernelI((?:Li-?\d+E){8})Lb([01])E", name)
    return bool(m) and m.group(2) == "1"


def test_reports_are_current():
    reports = glob.glob(os.path.join(OBJ_DIR, "*.resources.txt"))
    if not reports:
        pytest.skip("library not built (run __graft_entry__.build() first)")
    newest_src = max(os.path.getmtime(p) for p in glob.glob(os.path.join(PKG, "csrc", "*")))
    stale = [p for p in reports if os.path.getmtime(p) < newest_src]
    assert not stale, f"resource reports older than the sources (rebuild): {stale}"


def test_product_kernels_spill_free_and_two_waves():
    ks = _kernels()
    if not ks:
        pytest.skip("library not built (run __graft_entry__.build() first)")
    gemm = [n for n in ks if "w4a8_gemm_kernel" in n]
    assert len(gemm) > 100          # every row source x group size x tile body
    bad = []
    for name, r in ks.items():
        if _is_debug(name):
            continue
        if r.get("ScratchSize", 0) != 0 or r.get("Occupancy", 0) < 2:
            bad.append((r["file"], name, r))
    assert not bad, "kernels with scratch or one wave per SIMD:\n" + "\n".join(map(str, bad))


def test_debug_kernels_are_recognised():
    ks = _kernels()
    if not ks:
        pytest.skip("library not built")
    debug = [n for n in ks if _is_debug(n)]
    # the three debug sources instantiate the same tile bodies as the product
    assert debug and all(ks[n]["file"].startswith("gemm_debug") for n in debug)
    assert not any(_is_debug(n) for n in ks if ks[n]["file"] in ("gemm_routed.resources.txt",
                                                                  "gemm_csr.resources.txt"))


LLVM_BIN = "/opt/rocm/llvm/bin"


def _calls_in_object(obj, tmp):
    """Number of s_swappc_b64 (function calls) in the gfx950 code object of
    one built object file (its .hip_fatbin section, unbundled). Long branches
    (s_getpc / s_setpc) are not calls and are not counted."""
    import subprocess
    base = os.path.join(tmp, os.path.basename(obj))
    subprocess.run([f"{LLVM_BIN}/llvm-objcopy", f"--dump-section=.hip_fatbin={base}.fatbin", obj], check=True)
    subprocess.run([f"{LLVM_BIN}/clang-offload-bundler", "--type=o", "--targets=hipv4-amdgcn-amd-amdhsa--gfx950",
                    f"--input={base}.fatbin", f"--output={base}.co", "--unbundle"], check=True)
    dis = subprocess.run([f"{LLVM_BIN}/llvm-objdump", "-d", f"{base}.co"], check=True, capture_output=True,
                         text=True).stdout
    return dis.count("s_swappc_b64")


def test_no_kernel_calls_a_function(tmp_path):
    """Every tile body is inlined into its kernel. A tile body the compiler
    left as a called function (kernel arguments through scratch, its barriers
    and LDS in the callee) hung the GPU; the lambdas on the tile path are
    always_inline, and this checks the code objects for any call."""
    objs = sorted(glob.glob(os.path.join(OBJ_DIR, "gemm_*.o")))
    if not objs or not os.path.exists(f"{LLVM_BIN}/llvm-objdump"):
        pytest.skip("library not built or ROCm LLVM tools absent")
    from concurrent.futures import ThreadPoolExecutor
    with ThreadPoolExecutor(max_workers=min(len(objs), 6)) as ex:
        calls = dict(zip(objs, ex.map(lambda o: _calls_in_object(o, str(tmp_path)), objs)))
    bad = {os.path.basename(o): n for o, n in calls.items() if n}
    assert not bad, f"function calls in GEMM code objects: {bad}"
