"""ctypes binding of the C ABI declared in include/fa_mi355x.h.

This is the binding a Python caller without the torch extension would write;
the tests use it to load libfa_mi355x.so directly, check its exported
symbols and validation branches on the CPU, and drive fa_fwd on the GPU with
raw device pointers.
"""
from __future__ import annotations

import ctypes
import os
import re

REPO_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO_ROOT, "include", "fa_mi355x.h")
# FA_MI355X_LIB: another build of the library to test (tests/test_abi_asan.py
# points it at an AddressSanitizer build of the host code).
LIB_PATH = os.environ.get("FA_MI355X_LIB") or os.path.join(
    REPO_ROOT, "flash-attention_amd", "flash_attention_runtime", "libfa_mi355x.so")
# The LDS-poison debug build of the same library (flash-attention_amd/build.py).
POISON_LIB_PATH = os.path.join(
    REPO_ROOT, "flash-attention_amd", "flash_attention_runtime", "libfa_mi355x_poison.so")
# The build whose fp16 8-wave non-causal kernel keeps the 32x32x16 MFMA form.
MFMA32_LIB_PATH = os.path.join(
    REPO_ROOT, "flash-attention_amd", "flash_attention_runtime", "libfa_mi355x_mfma32.so")

FA_OK, FA_ERR_NULL, FA_ERR_DTYPE, FA_ERR_SHAPE, FA_ERR_HEADDIM, FA_ERR_STRIDE, \
    FA_ERR_UNSUPPORTED, FA_ERR_HIP, FA_ERR_ARG = range(9)
FA_DTYPE_F16, FA_DTYPE_BF16 = 0, 1
FA_SCRATCH_BYTES = 32 << 20  # include/fa_mi355x.h


class FaFwdParams(ctypes.Structure):
    _fields_ = [
        ("q", ctypes.c_void_p),
        ("k", ctypes.c_void_p),
        ("v", ctypes.c_void_p),
        ("o", ctypes.c_void_p),
        ("lse", ctypes.POINTER(ctypes.c_float)),
        ("q_stride", ctypes.c_int64 * 3),
        ("k_stride", ctypes.c_int64 * 3),
        ("v_stride", ctypes.c_int64 * 3),
        ("o_stride", ctypes.c_int64 * 3),
        ("batch", ctypes.c_int32),
        ("heads", ctypes.c_int32),
        ("seq_len", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("softmax_scale", ctypes.c_float),
        ("causal", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
    ]


class FaDeviceInfo(ctypes.Structure):
    _fields_ = [
        ("name", ctypes.c_char * 256),
        ("arch", ctypes.c_char * 64),
        ("compute_units", ctypes.c_int32),
        ("clock_khz", ctypes.c_int32),
        ("lds_per_cu_bytes", ctypes.c_int64),
        ("l2_bytes", ctypes.c_int64),
        ("memory_bus_width_bits", ctypes.c_int32),
        ("memory_clock_khz", ctypes.c_int32),
        ("fp16_dense_peak_tflops", ctypes.c_double),
        ("hbm_peak_gbps", ctypes.c_double),
        ("global_mem_bytes", ctypes.c_int64),
        ("lds_per_block_bytes", ctypes.c_int64),
        ("regs_per_block", ctypes.c_int32),
        ("regs_per_cu", ctypes.c_int32),
        ("max_threads_per_cu", ctypes.c_int32),
        ("max_threads_per_block", ctypes.c_int32),
        ("wavefront_size", ctypes.c_int32),
        ("arch_major", ctypes.c_int32),
        ("arch_minor", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
    ]


FA_PLAN_MAX_ITEMS = 128


class FaFwdPlan(ctypes.Structure):
    _fields_ = [
        ("block_rows", ctypes.c_int32),
        ("n_items", ctypes.c_int32),
        ("n_slots", ctypes.c_int32),
        ("n_merge", ctypes.c_int32),
        ("xcd_heads", ctypes.c_int32),
        ("key_halves", ctypes.c_int32),
        ("head_group", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("workspace_bytes", ctypes.c_uint64),
        ("q_tile", ctypes.c_int32 * FA_PLAN_MAX_ITEMS),
        ("tile_begin", ctypes.c_int32 * FA_PLAN_MAX_ITEMS),
        ("tile_end", ctypes.c_int32 * FA_PLAN_MAX_ITEMS),
        ("n_chunks", ctypes.c_int32 * FA_PLAN_MAX_ITEMS),
        ("slot", ctypes.c_int32 * FA_PLAN_MAX_ITEMS),
        ("head", ctypes.c_int32 * FA_PLAN_MAX_ITEMS),
    ]


def declared_functions(header: str = HEADER) -> list[str]:
    """Names of the functions declared in the public header."""
    text = open(header).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\**\s+\**(fa_\w+)\s*\(", text, re.M)))


def load(path: str = LIB_PATH):
    L = ctypes.CDLL(path)
    P = ctypes.POINTER(FaFwdParams)
    L.fa_fwd_validate.argtypes = [P]
    L.fa_fwd_validate.restype = ctypes.c_int
    L.fa_fwd.argtypes = [P, ctypes.c_void_p]
    L.fa_fwd.restype = ctypes.c_int
    L.fa_fwd_timed.argtypes = [P, ctypes.c_void_p, ctypes.POINTER(ctypes.c_float)]
    L.fa_fwd_timed.restype = ctypes.c_int
    L.fa_fwd_workspace_size.argtypes = [P, ctypes.POINTER(ctypes.c_uint64)]
    L.fa_fwd_workspace_size.restype = ctypes.c_int
    L.fa_fwd_ws.argtypes = [P, ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p]
    L.fa_fwd_ws.restype = ctypes.c_int
    L.fa_fwd_ws_timed.argtypes = [P, ctypes.c_void_p, ctypes.c_uint64, ctypes.c_void_p,
                                  ctypes.POINTER(ctypes.c_float)]
    L.fa_fwd_ws_timed.restype = ctypes.c_int
    L.fa_fwd_scratch.argtypes = [P, ctypes.c_void_p]
    L.fa_fwd_scratch.restype = ctypes.c_int
    L.fa_fwd_plan.argtypes = [P, ctypes.c_int32, ctypes.POINTER(FaFwdPlan)]
    L.fa_fwd_plan.restype = ctypes.c_int
    L.fa_status_str.argtypes = [ctypes.c_int]
    L.fa_status_str.restype = ctypes.c_char_p
    L.fa_last_error.argtypes = []
    L.fa_last_error.restype = ctypes.c_char_p
    L.fa_device_info.argtypes = [ctypes.c_int, ctypes.POINTER(FaDeviceInfo)]
    L.fa_device_info.restype = ctypes.c_int
    L.fa_version.argtypes = []
    L.fa_version.restype = ctypes.c_char_p
    return L


def params_from_tensors(q, k, v, o, lse=None, causal=False, scale=None):
    """Fills FaFwdParams from torch tensors [B, H, N, D] (device pointers)."""
    import math

    import torch

    p = FaFwdParams()
    p.q, p.k, p.v, p.o = q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr()
    p.lse = ctypes.cast(lse.data_ptr(), ctypes.POINTER(ctypes.c_float)) if lse is not None else None
    for name, t in (("q_stride", q), ("k_stride", k), ("v_stride", v), ("o_stride", o)):
        arr = getattr(p, name)
        for i in range(3):
            arr[i] = t.stride(i)
    p.batch, p.heads, p.seq_len, p.head_dim = (int(x) for x in q.shape)
    p.softmax_scale = 1.0 / math.sqrt(q.shape[3]) if scale is None else float(scale)
    p.causal = 1 if causal else 0
    p.dtype = FA_DTYPE_BF16 if q.dtype == torch.bfloat16 else FA_DTYPE_F16
    return p
