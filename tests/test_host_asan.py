"""AddressSanitizer build of the host C-ABI code (no GPU needed).

``csrc/api.hip`` -- argument validation, tile selection, workspace carving,
the CPU self-test -- is compiled with ``-fsanitize=address`` on its host pass
only (``-Xarch_host``; the device code is not instrumented) and linked with
the library's other objects and ``tests/asan/host_abi_driver.cpp`` into an
executable that calls every entry point on its rejection paths, the size
helpers and the self-test. Any out-of-bounds or use-after-free access in that
host code aborts the run."""

import glob
import os
import shutil
import subprocess

import pytest

from conftest import ROOT

PKG = os.path.join(ROOT, "flagos-kernel-gen_amd")
OBJ_DIR = os.path.join(PKG, "_build")


def _hipcc():
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and os.path.exists(c):
            return c
    return None


def test_host_abi_under_address_sanitizer(tmp_path):
    hipcc = _hipcc()
    if hipcc is None:
        pytest.skip("hipcc not available")
    objs = [o for o in sorted(glob.glob(os.path.join(OBJ_DIR, "*.o"))) if os.path.basename(o) != "api.o"]
    if not objs:
        pytest.skip("library objects not built (run __graft_entry__.build() first)")
    api_o = str(tmp_path / "api_asan.o")
    exe = str(tmp_path / "host_abi_asan")
    flags = ["--offload-arch=gfx950", "-O1", "-g", "-std=c++17", "-fPIC",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fno-omit-frame-pointer"]
    r = subprocess.run([hipcc, "-x", "hip", *flags, "-c", os.path.join(PKG, "csrc", "api.hip"), "-o", api_o],
                       capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-3000:]
    # the driver is plain C++ (host compiler); the link pulls in the ASan runtime
    drv_o = str(tmp_path / "driver.o")
    r = subprocess.run(["g++", "-O1", "-g", "-fsanitize=address", "-fno-omit-frame-pointer", "-I",
                        os.path.join(ROOT, "include"), "-c", os.path.join(ROOT, "tests", "asan", "host_abi_driver.cpp"),
                        "-o", drv_o], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-3000:]
    r = subprocess.run([hipcc, "--offload-arch=gfx950", "-Xarch_host", "-fsanitize=address", drv_o, api_o, *objs,
                        "-o", exe], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stderr[-3000:]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:abort_on_error=1", HIP_VISIBLE_DEVICES="")
    r = subprocess.run([exe], capture_output=True, text=True, timeout=300, env=env)
    assert r.returncode == 0, (r.stdout + r.stderr)[-4000:]
    assert "host ABI checks passed" in r.stdout
