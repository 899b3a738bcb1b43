"""The C++ callers of the C ABI on the GPU.

- tests/cpp/fa_correctness: the counterpart of the reference's
  benchmark/cpp/correctness_v6.cu:106-217 (its N=64 single-tile case with
  check_close atol 2e-2 / rtol 8e-2 over every element, plus ragged, causal,
  bf16 and head_dim 64 cases against the fp64 oracle at the contract bars).
- flash_attention_runtime/fa_device_query: the counterpart of the
  reference's utils/get_gpu_hardware_param.cu:1-26, every field of it.
"""
from __future__ import annotations

import json
import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CORRECTNESS = os.path.join(REPO, "tests", "cpp", "fa_correctness")
QUERY = os.path.join(REPO, "flash-attention_amd", "flash_attention_runtime", "fa_device_query")


def test_cpp_correctness_executable():
    print("case fa_correctness", flush=True)
    r = subprocess.run([CORRECTNESS], capture_output=True, text=True, timeout=240)
    print(r.stdout[-3000:], flush=True)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    assert "ALL PASSED" in r.stdout
    assert "case reference_v6: B=1 H=1 N=64 D=128 fp16" in r.stdout
    assert "check_close(atol 2e-02, rtol 8e-02)" in r.stdout


def test_device_query_cli(fa):
    print("case fa_device_query", flush=True)
    text = subprocess.run([QUERY], capture_output=True, text=True, timeout=60, check=True).stdout
    for label in ("Global Memory:", "LDS per Block:", "LDS per CU:", "Registers per Block:",
                  "Registers per CU:", "L2 Cache Size:", "Arch (major.minor):", "CU Count:",
                  "Max Threads per CU:", "Max Threads per Block:"):
        assert label in text, label
    d = json.loads(subprocess.run([QUERY, "--json"], capture_output=True, text=True, timeout=60,
                                  check=True).stdout)
    info = fa.device_info(0)
    assert d["compute_units"] == info["compute_units"]
    assert d["global_mem_mb"] == info["global_mem_bytes"] >> 20
    assert d["wavefront_size"] == info["wavefront_size"] == 64
    assert info["max_threads_per_block"] >= 256 and info["regs_per_block"] > 0
    assert info["lds_per_block_bytes"] >= 64 * 1024
    if info["arch"].startswith("gfx950"):
        assert info["global_mem_bytes"] > 250 * 2**30  # 288 GB HBM3E
        assert (info["arch_major"], info["arch_minor"]) == (9, 5)
