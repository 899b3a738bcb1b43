"""Builds the MI355X FlashAttention-2 forward in-tree.

Outputs (next to the Python package, so they travel with the repository):
  flash_attention_runtime/libfa_mi355x.so   HIP kernels + C ABI (hipcc, gfx950)
  flash_attention_runtime/libfa_mi355x_poison.so   the same with LDS poisoning (tests only)
  flash_attention_runtime/libfa_mi355x_mfma32.so   the same with the 32x32x16 MFMA form of the
                                                   fp16 8-wave kernel (tests and counters only)
  flash_attention_runtime/_C<EXT_SUFFIX>     torch/pybind binding over the C ABI
  flash_attention_runtime/fa_profile         C++ benchmark CLI over the C ABI
  flash_attention_runtime/fa_device_query    device description CLI over the C ABI
  flash_attention_runtime/fa_mfma_probe      MFMA-only throughput probe (peak cross-check)

Replaces the reference's JIT build (python/flash_attention_runtime/
__init__.py:10-27, torch.utils.cpp_extension.load of _ext.cu with nvcc) by an
explicit ahead-of-time build: one HIP code path for gfx950, no CUDA headers.

Usage: python flash-attention_amd/build.py [--jobs N]
"""
from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor

PKG_ROOT = os.path.dirname(os.path.abspath(__file__))
REPO_ROOT = os.path.dirname(PKG_ROOT)
CSRC = os.path.join(PKG_ROOT, "csrc")
OUT_DIR = os.path.join(PKG_ROOT, "flash_attention_runtime")
INCLUDE = os.path.join(REPO_ROOT, "include")
BUILD_DIR = os.path.join(PKG_ROOT, "_build")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

ARCH = "gfx950"
# -packed-fp32-ops: keep the compiler from forming v_pk_{add,mul,fma}_f32.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        ln for ln in proc.stdout.splitlines()
        if "packed-fp32-ops" not in ln and "hip-link" not in ln
        and "not a recognized feature for this target" not in ln
    )
    if proc.returncode != 0:
        sys.stderr.write(out + "\n")
        raise RuntimeError(f"build step failed ({proc.returncode}): {' '.join(cmd)}")


def _hipcc() -> str:
    for cand in (os.path.join(ROCM, "bin", "hipcc"), shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found")


def build_hip_library(jobs: int) -> list[str]:
    """Compiles csrc/fa_fwd_kernel.hip (kernels and launch), fa_plan.cpp
    (host work planning) and fa_api.cpp (the C ABI) with hipcc and links the
    shared library libfa_mi355x.so.  The kernel source is compiled a second
    time with -DFA_LDS_POISON into the debug library
    libfa_mi355x_poison.so (same ABI; staged LDS is filled with NaN before
    every staging write), and a third time with -DFA_MFMA32 into
    libfa_mi355x_mfma32.so (same ABI; fp16 non-causal problems of the
    8-wave range run the 32x32x16 MFMA form of the kernel instead of the
    16x16x32 one), which only the tests and the counter comparison of the
    MFMA shapes load."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    hipcc = _hipcc()
    kernel = os.path.join(CSRC, "fa_fwd_kernel.hip")
    host = [os.path.join(CSRC, "fa_plan.cpp"), os.path.join(CSRC, "fa_api.cpp")]

    def obj_of(src: str, tag: str = "") -> str:
        return os.path.join(BUILD_DIR, os.path.basename(src) + tag + ".o")

    cmds = []
    for src in [kernel, *host]:
        lang = ["-x", "hip"] if src.endswith(".hip") else []
        cmds.append([hipcc, *HIP_FLAGS, "-I", INCLUDE, "-I", CSRC, *lang, "-c", src,
                     "-o", obj_of(src)])
    cmds.append([hipcc, *HIP_FLAGS, "-DFA_LDS_POISON", "-I", INCLUDE, "-I", CSRC, "-x", "hip",
                 "-c", kernel, "-o", obj_of(kernel, ".poison")])
    cmds.append([hipcc, *HIP_FLAGS, "-DFA_MFMA32", "-I", INCLUDE, "-I", CSRC, "-x", "hip",
                 "-c", kernel, "-o", obj_of(kernel, ".mfma32")])
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        list(ex.map(_run, cmds))
    libs = []
    for name, kobj in (("libfa_mi355x.so", obj_of(kernel)),
                       ("libfa_mi355x_poison.so", obj_of(kernel, ".poison")),
                       ("libfa_mi355x_mfma32.so", obj_of(kernel, ".mfma32"))):
        lib = os.path.join(OUT_DIR, name)
        _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", kobj,
              *[obj_of(h) for h in host], "-o", lib + ".tmp"])
        os.replace(lib + ".tmp", lib)
        libs.append(lib)
    return libs


def build_torch_binding() -> str:
    """Compiles the pybind/torch host binding (fa_torch_ext.cpp) with g++ and
    links it against libfa_mi355x.so (rpath $ORIGIN)."""
    import torch
    from torch.utils import cpp_extension

    torch_lib = os.path.join(os.path.dirname(torch.__file__), "lib")
    ext_suffix = sysconfig.get_config_var("EXT_SUFFIX") or ".so"
    out = os.path.join(OUT_DIR, "_C" + ext_suffix)
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    incs = [*cpp_extension.include_paths(), sysconfig.get_paths()["include"],
            os.path.join(ROCM, "include"), INCLUDE]
    cmd = [
        "g++", "-O2", "-std=c++17", "-fPIC", "-shared", "-w",
        "-DTORCH_EXTENSION_NAME=_C", "-DTORCH_API_INCLUDE_EXTENSION_H",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
        *[f"-I{p}" for p in incs],
        os.path.join(CSRC, "fa_torch_ext.cpp"),
        f"-L{OUT_DIR}", "-lfa_mi355x",
        f"-L{torch_lib}", "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python", "-lc10_hip",
        "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{torch_lib}",
        "-o", out + ".tmp",
    ]
    _run(cmd)
    os.replace(out + ".tmp", out)
    return out


def build_profile_cli() -> str:
    """Links the fa_profile executable (csrc/fa_profile.cpp) against
    libfa_mi355x.so (rpath $ORIGIN)."""
    out = os.path.join(OUT_DIR, "fa_profile")
    _run([_hipcc(), "-O2", "-std=c++17", "-Wall", "-I", INCLUDE,
          os.path.join(CSRC, "fa_profile.cpp"), f"-L{OUT_DIR}", "-lfa_mi355x",
          "-Wl,-rpath,$ORIGIN", "-o", out + ".tmp"])
    os.replace(out + ".tmp", out)
    return out


def build_device_query() -> str:
    """Links the fa_device_query executable (csrc/fa_device_query.cpp)
    against libfa_mi355x.so (rpath $ORIGIN)."""
    out = os.path.join(OUT_DIR, "fa_device_query")
    _run([_hipcc(), "-O2", "-std=c++17", "-Wall", "-I", INCLUDE,
          os.path.join(CSRC, "fa_device_query.cpp"), f"-L{OUT_DIR}", "-lfa_mi355x",
          "-Wl,-rpath,$ORIGIN", "-o", out + ".tmp"])
    os.replace(out + ".tmp", out)
    return out


def build_mfma_probe() -> str:
    """Builds the fa_mfma_probe executable (csrc/fa_mfma_probe.hip), which
    times MFMA-only waves to cross-check the computed MFMA peak."""
    out = os.path.join(OUT_DIR, "fa_mfma_probe")
    _run([_hipcc(), *[f for f in HIP_FLAGS if f != "-fPIC"],
          os.path.join(CSRC, "fa_mfma_probe.hip"), "-o", out + ".tmp"])
    os.replace(out + ".tmp", out)
    return out


def build(jobs: int = 8) -> list[str]:
    libs = build_hip_library(jobs)
    ext = build_torch_binding()
    cli = build_profile_cli()
    query = build_device_query()
    probe = build_mfma_probe()
    return [*libs, ext, cli, query, probe]


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--jobs", type=int, default=8)
    args = ap.parse_args()
    for path in build(args.jobs):
        print("built", os.path.relpath(path, REPO_ROOT))


if __name__ == "__main__":
    main()
