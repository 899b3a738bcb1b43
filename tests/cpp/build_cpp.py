"""Builds tests/cpp/fa_correctness (the C++ correctness executable over the C
ABI; test infrastructure, not product).  Needs the library
(flash-attention_amd/build.py) and the oracle (oracle/oracle.py build())."""
from __future__ import annotations

import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
LIBDIR = os.path.join(REPO, "flash-attention_amd", "flash_attention_runtime")
ORACLE = os.path.join(REPO, "oracle")
SRC = os.path.join(HERE, "fa_correctness.cpp")
EXE = os.path.join(HERE, "fa_correctness")


def build() -> str:
    hipcc = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "bin", "hipcc")
    tmp = EXE + ".tmp"
    cmd = [hipcc, "-O2", "-std=c++17", "-Wall", "-I", os.path.join(REPO, "include"), "-I", ORACLE,
           SRC, f"-L{LIBDIR}", "-lfa_mi355x", f"-L{ORACLE}", "-l:liboracle.so",
           f"-Wl,-rpath,{os.path.relpath(LIBDIR, HERE).join(['$ORIGIN/', ''])}",
           f"-Wl,-rpath,{os.path.relpath(ORACLE, HERE).join(['$ORIGIN/', ''])}", "-o", tmp]
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if proc.returncode != 0:
        raise RuntimeError(proc.stdout)
    os.replace(tmp, EXE)
    return EXE


if __name__ == "__main__":
    print(build())
