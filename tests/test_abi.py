"""CPU tests of the drop-in boundary: the C ABI in include/fa_mi355x.h as
exported by libfa_mi355x.so, and the host-side checks of the torch binding.

Nothing here launches a kernel.  fa_fwd_validate is pure host code, so every
rejection rule is exercised with fake (never dereferenced) device addresses;
fa_fwd / fa_fwd_timed are called only with arguments that validation rejects
before any HIP call.  The rules mirror the reference's validate_inputs /
check_cuda_tensor (python/flash_attention_runtime/_ext.cu:19-57) where they
coincide, and otherwise the kernel's own limits.
"""
from __future__ import annotations

import ctypes
import json
import math
import os
import subprocess
import sys

import pytest

import abi_ctypes as A

HERE = os.path.dirname(os.path.abspath(__file__))

# Fake device addresses: 16-byte aligned, never dereferenced by validation.
QA, KA, VA, OA, LA = 0x10000, 0x20000, 0x30000, 0x40000, 0x50000


@pytest.fixture(scope="module")
def lib():
    return A.load()


def contiguous(B=2, H=4, N=256, D=128, dtype=A.FA_DTYPE_F16, causal=0, lse=True):
    p = A.FaFwdParams()
    p.q, p.k, p.v, p.o = QA, KA, VA, OA
    p.lse = ctypes.cast(LA, ctypes.POINTER(ctypes.c_float)) if lse else None
    st = (H * N * D, N * D, D)
    for name in ("q_stride", "k_stride", "v_stride", "o_stride"):
        arr = getattr(p, name)
        for i in range(3):
            arr[i] = st[i]
    p.batch, p.heads, p.seq_len, p.head_dim = B, H, N, D
    p.softmax_scale = 1.0 / math.sqrt(D)
    p.causal = causal
    p.dtype = dtype
    return p


def check(lib, p, expect, msg=None):
    rc = lib.fa_fwd_validate(ctypes.byref(p))
    err = lib.fa_last_error().decode()
    assert rc == expect, (rc, err)
    if msg is not None:
        assert msg in err, err
    if expect == A.FA_OK:
        assert err == ""


# ---------------------------------------------------------------- exports


def test_every_declared_function_is_exported(lib):
    names = A.declared_functions()
    assert set(names) >= {"fa_fwd", "fa_fwd_validate", "fa_fwd_timed", "fa_status_str",
                          "fa_last_error", "fa_device_info", "fa_version", "fa_fwd_ws",
                          "fa_fwd_ws_timed", "fa_fwd_workspace_size", "fa_fwd_plan"}
    for n in names:
        assert hasattr(lib, n), f"{n} declared in include/fa_mi355x.h but not exported"


def test_exported_symbols_are_c_linkage():
    out = subprocess.run(["nm", "-D", "--defined-only", A.LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    for n in A.declared_functions():
        assert n in exported, f"{n} is not an unmangled text symbol"


def test_poison_build_exports_the_same_abi():
    """The LDS-poison debug library (tests only) is built beside the product
    one, loads on a host without a GPU, and exports every declared function
    unmangled, so any test can run against it in place of the product."""
    if not os.path.exists(A.POISON_LIB_PATH):
        pytest.skip("run build() first: no LDS-poison library")
    L = A.load(A.POISON_LIB_PATH)
    out = subprocess.run(["nm", "-D", "--defined-only", A.POISON_LIB_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    for n in A.declared_functions():
        assert hasattr(L, n) and n in exported, n


def test_mfma32_build_exports_the_same_abi():
    """The 32x32x16-MFMA test library exports the same ABI and loads on a
    host without a GPU."""
    if not os.path.exists(A.MFMA32_LIB_PATH):
        pytest.skip("run build() first: no 32x32x16 library")
    L = A.load(A.MFMA32_LIB_PATH)
    for n in A.declared_functions():
        assert hasattr(L, n), n


def test_status_enum_matches_header():
    text = open(A.HEADER).read()
    import re

    vals = dict((k, int(v)) for k, v in re.findall(r"(FA_(?:OK|ERR_\w+))\s*=\s*(\d+)", text))
    assert vals == {"FA_OK": A.FA_OK, "FA_ERR_NULL": A.FA_ERR_NULL, "FA_ERR_DTYPE": A.FA_ERR_DTYPE,
                    "FA_ERR_SHAPE": A.FA_ERR_SHAPE, "FA_ERR_HEADDIM": A.FA_ERR_HEADDIM,
                    "FA_ERR_STRIDE": A.FA_ERR_STRIDE, "FA_ERR_UNSUPPORTED": A.FA_ERR_UNSUPPORTED,
                    "FA_ERR_HIP": A.FA_ERR_HIP, "FA_ERR_ARG": A.FA_ERR_ARG}
    d = dict((k, int(v)) for k, v in re.findall(r"(FA_DTYPE_\w+)\s*=\s*(\d+)", text))
    assert d == {"FA_DTYPE_F16": A.FA_DTYPE_F16, "FA_DTYPE_BF16": A.FA_DTYPE_BF16}


LAYOUT_PROBE = r"""
#include <stddef.h>
#include <stdio.h>
#include "fa_mi355x.h"
#define F(T, m) printf("\"%s.%s\": [%zu, %zu],", #T, #m, offsetof(T, m), sizeof(((T*)0)->m))
int main(void) {
  printf("{");
  F(fa_fwd_params, q); F(fa_fwd_params, k); F(fa_fwd_params, v); F(fa_fwd_params, o);
  F(fa_fwd_params, lse); F(fa_fwd_params, q_stride); F(fa_fwd_params, k_stride);
  F(fa_fwd_params, v_stride); F(fa_fwd_params, o_stride); F(fa_fwd_params, batch);
  F(fa_fwd_params, heads); F(fa_fwd_params, seq_len); F(fa_fwd_params, head_dim);
  F(fa_fwd_params, softmax_scale); F(fa_fwd_params, causal); F(fa_fwd_params, dtype);
  F(fa_device_info_t, name); F(fa_device_info_t, arch); F(fa_device_info_t, compute_units);
  F(fa_device_info_t, clock_khz); F(fa_device_info_t, lds_per_cu_bytes);
  F(fa_device_info_t, l2_bytes); F(fa_device_info_t, memory_bus_width_bits);
  F(fa_device_info_t, memory_clock_khz); F(fa_device_info_t, fp16_dense_peak_tflops);
  F(fa_device_info_t, hbm_peak_gbps); F(fa_device_info_t, global_mem_bytes);
  F(fa_device_info_t, lds_per_block_bytes); F(fa_device_info_t, regs_per_block);
  F(fa_device_info_t, regs_per_cu); F(fa_device_info_t, max_threads_per_cu);
  F(fa_device_info_t, max_threads_per_block); F(fa_device_info_t, wavefront_size);
  F(fa_device_info_t, arch_major); F(fa_device_info_t, arch_minor); F(fa_device_info_t, reserved);
  F(fa_fwd_plan_t, block_rows); F(fa_fwd_plan_t, n_items); F(fa_fwd_plan_t, n_slots);
  F(fa_fwd_plan_t, n_merge); F(fa_fwd_plan_t, xcd_heads); F(fa_fwd_plan_t, key_halves);
  F(fa_fwd_plan_t, head_group); F(fa_fwd_plan_t, reserved);
  F(fa_fwd_plan_t, workspace_bytes);
  F(fa_fwd_plan_t, q_tile); F(fa_fwd_plan_t, tile_begin); F(fa_fwd_plan_t, tile_end);
  F(fa_fwd_plan_t, n_chunks); F(fa_fwd_plan_t, slot); F(fa_fwd_plan_t, head);
  printf("\"sizeof.fa_fwd_params\": [%zu, 0], \"sizeof.fa_device_info_t\": [%zu, 0], "
         "\"sizeof.fa_fwd_plan_t\": [%zu, 0]}\n",
         sizeof(fa_fwd_params), sizeof(fa_device_info_t), sizeof(fa_fwd_plan_t));
  return 0;
}
"""


def test_ctypes_struct_layout_matches_c(tmp_path):
    """The ctypes mirror of the structs (the binding a Python caller uses)
    has the same offsets and sizes as the C compiler gives the header."""
    src = tmp_path / "probe.c"
    exe = tmp_path / "probe"
    src.write_text(LAYOUT_PROBE)
    subprocess.run(["gcc", "-std=c99", "-I", os.path.dirname(A.HEADER), str(src), "-o", str(exe)],
                   check=True)
    c = json.loads(subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout)
    for cls, cname in ((A.FaFwdParams, "fa_fwd_params"), (A.FaDeviceInfo, "fa_device_info_t"),
                       (A.FaFwdPlan, "fa_fwd_plan_t")):
        for fname, _ in cls._fields_:
            off, size = c[f"{cname}.{fname}"]
            desc = getattr(cls, fname)
            assert (desc.offset, desc.size) == (off, size), (cname, fname)
        assert ctypes.sizeof(cls) == c[f"sizeof.{cname}"][0]


# ---------------------------------------------------------------- status strings


def test_status_strings(lib):
    seen = set()
    for s in range(9):
        t = lib.fa_status_str(s).decode()
        assert t and t not in seen
        seen.add(t)
    assert lib.fa_status_str(0).decode() == "ok"
    assert lib.fa_status_str(99).decode() == "unknown status"
    assert lib.fa_version().decode().startswith("fa_mi355x ")


# ---------------------------------------------------------------- validation


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("dtype", [A.FA_DTYPE_F16, A.FA_DTYPE_BF16])
@pytest.mark.parametrize("causal", [0, 1])
def test_valid_params_accepted(lib, D, dtype, causal):
    check(lib, contiguous(D=D, dtype=dtype, causal=causal), A.FA_OK)


@pytest.mark.parametrize("N", [1, 2, 31, 129, 3000, 4097])
def test_any_seq_len_accepted(lib, N):
    """Unlike the reference pybind path (seq_len % BlockM == 0, _ext.cu:49),
    every seq_len >= 1 is supported (ragged tails are masked)."""
    check(lib, contiguous(N=N), A.FA_OK)


def test_lse_optional(lib):
    check(lib, contiguous(lse=False), A.FA_OK)


def test_null_params(lib):
    assert lib.fa_fwd_validate(None) == A.FA_ERR_NULL
    assert "params" in lib.fa_last_error().decode()


@pytest.mark.parametrize("field", ["q", "k", "v", "o"])
def test_null_tensor(lib, field):
    p = contiguous()
    setattr(p, field, None)
    check(lib, p, A.FA_ERR_NULL, f"{field} is NULL")


@pytest.mark.parametrize("dtype", [-1, 2, 7])
def test_bad_dtype(lib, dtype):
    check(lib, contiguous(dtype=dtype), A.FA_ERR_DTYPE)


@pytest.mark.parametrize("field", ["batch", "heads", "seq_len"])
@pytest.mark.parametrize("val", [0, -3])
def test_bad_shape(lib, field, val):
    p = contiguous()
    setattr(p, field, val)
    check(lib, p, A.FA_ERR_SHAPE)


@pytest.mark.parametrize("D", [0, 32, 96, 127, 256])
def test_bad_head_dim(lib, D):
    """Reference: 'Only head_dim 128 is supported' (_ext.cu:45); here 64 and
    128 are supported and the message keeps the reference's wording."""
    p = contiguous(D=128)
    p.head_dim = D
    check(lib, p, A.FA_ERR_HEADDIM, "Only head_dim 64 and 128 are supported")


@pytest.mark.parametrize("causal", [-1, 2])
def test_bad_causal(lib, causal):
    check(lib, contiguous(causal=causal), A.FA_ERR_ARG, "causal")


@pytest.mark.parametrize("scale", [0.0, -0.125, float("inf"), float("nan"), float("-inf")])
def test_bad_scale(lib, scale):
    p = contiguous()
    p.softmax_scale = scale
    check(lib, p, A.FA_ERR_ARG, "softmax_scale")


@pytest.mark.parametrize("name", ["q_stride", "k_stride", "v_stride", "o_stride"])
@pytest.mark.parametrize("i", [0, 1, 2])
def test_stride_rules(lib, name, i):
    p = contiguous()
    getattr(p, name)[i] = -getattr(p, name)[i]
    check(lib, p, A.FA_ERR_STRIDE, "negative")
    p = contiguous()
    getattr(p, name)[i] += 4  # not a multiple of 8 elements
    check(lib, p, A.FA_ERR_STRIDE, "multiple of 8")


def test_overlapping_rows_rejected_but_single_row_ok(lib):
    p = contiguous(N=16)
    p.k_stride[2] = 64  # < head_dim 128
    check(lib, p, A.FA_ERR_STRIDE, "smaller than head_dim")
    p = contiguous(N=1)
    p.k_stride[2] = 0  # one row: the seq stride is never used
    check(lib, p, A.FA_OK)


def test_strided_views_accepted(lib):
    """BNHD storage seen as [B, H, N, D] (strides N*H*D, D, H*D) needs no copy."""
    B, H, N, D = 2, 4, 100, 64
    p = contiguous(B=B, H=H, N=N, D=D)
    for name in ("q_stride", "k_stride", "v_stride", "o_stride"):
        arr = getattr(p, name)
        arr[0], arr[1], arr[2] = N * H * D, D, H * D
    check(lib, p, A.FA_OK)
    p.q_stride[2] = 32  # rows of 64 elements 32 apart would overlap
    check(lib, p, A.FA_ERR_STRIDE, "smaller than head_dim")


@pytest.mark.parametrize("field", ["q", "k", "v", "o"])
def test_misaligned_pointer(lib, field):
    p = contiguous()
    setattr(p, field, getattr(p, field) + 8)
    check(lib, p, A.FA_ERR_STRIDE, "16-byte aligned")


def test_misaligned_lse(lib):
    p = contiguous()
    p.lse = ctypes.cast(LA + 2, ctypes.POINTER(ctypes.c_float))
    check(lib, p, A.FA_ERR_STRIDE, "lse")


def test_seq_stride_limit(lib):
    p = contiguous(N=16, D=64)
    p.v_stride[2] = 1 << 24
    check(lib, p, A.FA_OK)
    p.v_stride[2] = (1 << 24) + 8
    check(lib, p, A.FA_ERR_UNSUPPORTED, "v seq stride")


def test_grid_limit(lib):
    ok = contiguous(B=1 << 15, H=1 << 15, N=128, D=64)  # 2^30 workgroups
    check(lib, ok, A.FA_OK)
    big = contiguous(B=1 << 16, H=1 << 15, N=128, D=64)  # 2^31 workgroups
    check(lib, big, A.FA_ERR_UNSUPPORTED, "2^31-1")


def test_error_string_cleared_on_success(lib):
    check(lib, contiguous(dtype=5), A.FA_ERR_DTYPE)
    assert lib.fa_last_error().decode() != ""
    check(lib, contiguous(), A.FA_OK)


def test_first_failing_rule_wins(lib):
    p = contiguous(dtype=9)
    p.q = None
    check(lib, p, A.FA_ERR_NULL)


# ------------------------------------------- entry points reject before any HIP call


def test_fwd_rejects_before_launch(lib):
    assert lib.fa_fwd(None, None) == A.FA_ERR_NULL
    p = contiguous(D=96)
    p.head_dim = 96
    assert lib.fa_fwd(ctypes.byref(p), None) == A.FA_ERR_HEADDIM


def test_fwd_timed_rejects_before_launch(lib):
    ms = ctypes.c_float(-1.0)
    p = contiguous()
    assert lib.fa_fwd_timed(ctypes.byref(p), None, None) == A.FA_ERR_NULL
    p.softmax_scale = -1.0
    assert lib.fa_fwd_timed(ctypes.byref(p), None, ctypes.byref(ms)) == A.FA_ERR_ARG
    assert ms.value == 0.0  # *ms is reset on every call that gets that far


def test_fwd_ws_rejects_before_launch(lib):
    p = contiguous(D=96)
    p.head_dim = 96
    assert lib.fa_fwd_ws(ctypes.byref(p), None, 0, None) == A.FA_ERR_HEADDIM
    # a size without a buffer is rejected before anything else
    assert lib.fa_fwd_ws(ctypes.byref(contiguous()), None, 4096, None) == A.FA_ERR_NULL
    assert "workspace is NULL" in lib.fa_last_error().decode()
    ms = ctypes.c_float(-1.0)
    assert lib.fa_fwd_ws_timed(ctypes.byref(contiguous()), None, 16, None,
                               ctypes.byref(ms)) == A.FA_ERR_NULL
    assert ms.value == 0.0
    size = ctypes.c_uint64(7)
    assert lib.fa_fwd_workspace_size(ctypes.byref(p), ctypes.byref(size)) == A.FA_ERR_HEADDIM
    assert size.value == 0
    assert lib.fa_fwd_workspace_size(ctypes.byref(contiguous()), None) == A.FA_ERR_NULL


def test_device_info_null(lib):
    assert lib.fa_device_info(0, None) == A.FA_ERR_NULL


# ---------------------------------------------------------------- torch binding (host side)


@pytest.fixture(scope="module")
def rt():
    import flash_attention_runtime

    return flash_attention_runtime


def test_runtime_api_surface(rt):
    """Same public names as the reference package
    (python/flash_attention_runtime/__init__.py)."""
    for name in ("forward", "forward_timed", "device_info", "version"):
        assert callable(getattr(rt, name))
    assert rt.version().startswith("fa_mi355x ")


def test_runtime_rejects_cpu_tensors(rt):
    import torch

    q = torch.zeros(1, 1, 128, 128, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="q must be a CUDA tensor"):
        rt.forward(q, q, q)


def test_runtime_product_path_has_no_cpu_fallback():
    """The package imports only the HIP extension; with it missing the import
    fails loudly instead of falling back to another implementation."""
    code = ("import sys, importlib.abc\n"
            "class Block(importlib.abc.MetaPathFinder):\n"
            "    def find_spec(self, name, path, target=None):\n"
            "        if name == 'flash_attention_runtime._C': raise ImportError('blocked')\n"
            "sys.meta_path.insert(0, Block())\n"
            f"sys.path.insert(0, {os.path.join(os.path.dirname(HERE), 'flash-attention_amd')!r})\n"
            "try:\n"
            "    import flash_attention_runtime\n"
            "except ImportError as e:\n"
            "    print('IMPORT-FAILED', e)\n"
            "else:\n"
            "    print('IMPORTED')\n")
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=120)
    assert "IMPORT-FAILED" in out.stdout, out.stdout + out.stderr


def test_last_error_is_thread_local(lib):
    """Each thread sees the detail of its own last failure (the only mutable
    global state of the library is this thread-local string)."""
    import threading

    results = {}

    def worker(idx):
        p = contiguous(dtype=idx + 10) if idx % 2 else contiguous(D=128)
        if idx % 2 == 0:
            p.head_dim = 96
        for _ in range(200):
            rc = lib.fa_fwd_validate(ctypes.byref(p))
            msg = lib.fa_last_error().decode()
            ok = (rc == A.FA_ERR_DTYPE and f"dtype {idx + 10}" in msg) if idx % 2 else \
                 (rc == A.FA_ERR_HEADDIM and "got 96" in msg)
            if not ok:
                results[idx] = (rc, msg)
                return
        results[idx] = "ok"

    threads = [threading.Thread(target=worker, args=(i,)) for i in range(8)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert all(v == "ok" for v in results.values()), results
