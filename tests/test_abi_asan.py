"""The host layer of the library under AddressSanitizer, on the CPU.

fa_api.cpp (the C ABI: validation, status and error strings, workspace
sizing) and fa_plan.cpp (the split-KV and XCD placement planning, which fills
fixed-size tables) are compiled with g++ -fsanitize=address and linked with
the library's own kernel object into a separate libfa_mi355x.so; the CPU tests
of tests/test_abi.py (every validation branch) and tests/test_split_plan.py
(plans over the BASELINE configs and a sweep of shapes) then run against that
build in a child pytest with libasan preloaded.  Any invalid memory access
makes ASan abort the child with a report.  Needs the kernel object of a
previous build (flash-attention_amd/_build/fa_fwd_kernel.hip.o).
"""
from __future__ import annotations

import os
import subprocess
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(REPO, "flash-attention_amd", "csrc")
KERNEL_OBJ = os.path.join(REPO, "flash-attention_amd", "_build", "fa_fwd_kernel.hip.o")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")


def test_host_layer_under_asan(tmp_path):
    if not os.path.exists(KERNEL_OBJ):
        pytest.skip("kernel object not built (run flash-attention_amd/build.py)")
    lib = str(tmp_path / "libfa_mi355x.so")
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fPIC", "-shared", "-fsanitize=address",
           "-fno-omit-frame-pointer", "-D__HIP_PLATFORM_AMD__", "-I", os.path.join(ROCM, "include"),
           "-I", os.path.join(REPO, "include"), "-I", CSRC,
           os.path.join(CSRC, "fa_api.cpp"), os.path.join(CSRC, "fa_plan.cpp"), KERNEL_OBJ,
           f"-L{os.path.join(ROCM, 'lib')}", "-lamdhip64", "-o", lib]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-3000:]
    asan = subprocess.run(["g++", "-print-file-name=libasan.so"], capture_output=True, text=True,
                          check=True).stdout.strip()
    assert os.path.isabs(asan), asan
    env = dict(os.environ, FA_MI355X_LIB=lib, LD_PRELOAD=asan,
               ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:abort_on_error=1")
    child = [sys.executable, "-m", "pytest", "-q", "-x", "-s", "-p", "no:cacheprovider",
             "-m", "not gpu", "-k", "not runtime",
             os.path.join(HERE, "test_abi.py"), os.path.join(HERE, "test_split_plan.py")]
    r = subprocess.run(child, capture_output=True, text=True, env=env, cwd=REPO, timeout=600)
    print(r.stdout[-2000:])
    assert "AddressSanitizer" not in r.stderr + r.stdout, (r.stdout + r.stderr)[-4000:]
    assert r.returncode == 0, (r.stdout + r.stderr)[-4000:]
    assert " passed" in r.stdout
