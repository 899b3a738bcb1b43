"""ctypes wrapper of the CPU oracle (attn_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() as the
checker, and by bench.py for the timed CPU baseline.  The product package
(flash-attention_amd/) never imports it.

Inputs are numpy float32 arrays [B, H, N, D] holding fp16/bf16-quantised
values; see attn_oracle.c for which reference file each function restates.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_SRC = os.path.join(_HERE, "attn_oracle.c")

F16, BF16 = 0, 1
MUT_NONE, MUT_NO_SCALE, MUT_CAUSAL_DIAG, MUT_LSE_NO_MAX, MUT_TRANSPOSE_S, MUT_NO_NORMALISE = range(6)
MUTATIONS = {
    "no_scale": MUT_NO_SCALE,
    "causal_diag": MUT_CAUSAL_DIAG,
    "lse_no_max": MUT_LSE_NO_MAX,
    "transpose_s": MUT_TRANSPOSE_S,
    "no_normalise": MUT_NO_NORMALISE,
}

# x86-64-v3 (AVX2/FMA) rather than -march=native: the library is built here and
# also run on the GPU box's host CPU.
BUILD_FLAGS = ["-O3", "-march=x86-64-v3", "-fopenmp", "-fPIC", "-shared", "-std=gnu11",
               "-Wall", "-Wextra"]


def build() -> str:
    """Compiles attn_oracle.c into oracle/liboracle.so."""
    tmp = _LIB_PATH + ".tmp"
    cmd = ["gcc", *BUILD_FLAGS, _SRC, "-o", tmp, "-lm"]
    subprocess.run(cmd, check=True)
    os.replace(tmp, _LIB_PATH)
    return _LIB_PATH


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"oracle library missing: {_LIB_PATH} (run oracle.build())")
        L = ctypes.CDLL(_LIB_PATH)
        fp = ctypes.POINTER(ctypes.c_float)
        dp = ctypes.POINTER(ctypes.c_double)
        ip = ctypes.POINTER(ctypes.c_int32)
        up = ctypes.POINTER(ctypes.c_uint16)
        i32, i64, f32, f64 = ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_double
        L.oracle_attn_f64.argtypes = [fp, fp, fp, dp, dp, i32, i32, i32, i32, f64, i32, i32]
        L.oracle_attn_rows_f64.argtypes = [fp, fp, fp, i32, i32, i32, i32, f64, i32, i32,
                                           ip, ip, i64, dp, dp]
        L.oracle_ref_online_f32.argtypes = [fp, fp, fp, fp, i32, i32, i32, i32, f32, i32, i64, i64]
        L.oracle_kernel_numerics.argtypes = [fp, fp, fp, fp, fp, i32, i32, i32, i32, f32, i32,
                                             i32, i32]
        L.oracle_kernel_numerics_rows.argtypes = [fp, fp, fp, i32, i32, i32, i32, f32, i32, i32,
                                                  i32, ip, ip, i64, fp, fp]
        L.oracle_round_f16.argtypes = [fp, fp, up, i64]
        L.oracle_round_bf16.argtypes = [fp, fp, up, i64]
        L.oracle_num_threads.argtypes = []
        L.oracle_set_num_threads.argtypes = [i32]
        for name in ("oracle_attn_f64", "oracle_attn_rows_f64", "oracle_ref_online_f32",
                     "oracle_kernel_numerics", "oracle_kernel_numerics_rows",
                     "oracle_num_threads"):
            getattr(L, name).restype = ctypes.c_int
        _lib = L
    return _lib


def _f32(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    return a, a.ctypes.data_as(ctypes.POINTER(ctypes.c_float))


def _check_qkv(q, k, v):
    if q.ndim != 4 or q.shape != k.shape or q.shape != v.shape:
        raise ValueError(f"q, k, v must share a [B,H,N,D] shape, got {q.shape} {k.shape} {v.shape}")


def attn_f64(q, k, v, scale, causal=False, mutation=MUT_NONE):
    """Exact attention in float64: returns (o [B,H,N,D] f64, lse [B,H,N] f64)."""
    _check_qkv(q, k, v)
    B, H, N, D = q.shape
    q, qp = _f32(q)
    k, kp = _f32(k)
    v, vp = _f32(v)
    o = np.empty((B, H, N, D), np.float64)
    lse = np.empty((B, H, N), np.float64)
    rc = lib().oracle_attn_f64(qp, kp, vp, o.ctypes.data_as(ctypes.POINTER(ctypes.c_double)),
                               lse.ctypes.data_as(ctypes.POINTER(ctypes.c_double)),
                               B, H, N, D, float(scale), int(bool(causal)), int(mutation))
    if rc != 0:
        raise RuntimeError(f"oracle_attn_f64 failed: {rc}")
    return o, lse


def attn_rows_f64(q, k, v, scale, causal, sel_bh, sel_row, mutation=MUT_NONE):
    """Exact attention for selected rows (flattened head index bh = b*H + h,
    query row i).  Returns (o [n_sel, D] f64, lse [n_sel] f64)."""
    _check_qkv(q, k, v)
    B, H, N, D = q.shape
    q, qp = _f32(q)
    k, kp = _f32(k)
    v, vp = _f32(v)
    sel_bh = np.ascontiguousarray(sel_bh, dtype=np.int32)
    sel_row = np.ascontiguousarray(sel_row, dtype=np.int32)
    n = sel_bh.size
    o = np.empty((n, D), np.float64)
    lse = np.empty((n,), np.float64)
    ip = ctypes.POINTER(ctypes.c_int32)
    rc = lib().oracle_attn_rows_f64(qp, kp, vp, B, H, N, D, float(scale), int(bool(causal)),
                                    int(mutation), sel_bh.ctypes.data_as(ip),
                                    sel_row.ctypes.data_as(ip), n,
                                    o.ctypes.data_as(ctypes.POINTER(ctypes.c_double)),
                                    lse.ctypes.data_as(ctypes.POINTER(ctypes.c_double)))
    if rc != 0:
        raise RuntimeError(f"oracle_attn_rows_f64 failed: {rc}")
    return o, lse


def ref_online_f32(q, k, v, scale, causal=False, row_begin=0, row_end=None):
    """The reference CPU path (correctness_v6.cu:23-72), fp32 online softmax.
    Computes flattened rows [row_begin, row_end); other rows of the returned
    array are left as NaN."""
    _check_qkv(q, k, v)
    B, H, N, D = q.shape
    q, qp = _f32(q)
    k, kp = _f32(k)
    v, vp = _f32(v)
    total = B * H * N
    row_end = total if row_end is None else min(row_end, total)
    o = np.full((B, H, N, D), np.nan, np.float32)
    rc = lib().oracle_ref_online_f32(qp, kp, vp, o.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
                                     B, H, N, D, float(scale), int(bool(causal)), int(row_begin),
                                     int(row_end))
    if rc != 0:
        raise RuntimeError(f"oracle_ref_online_f32 failed: {rc}")
    return o


def kernel_numerics(q, k, v, scale, causal=False, dtype=F16, block_n=64):
    """Emulation of the reference kernel's arithmetic; returns (o f32 holding
    output-dtype values, lse f32)."""
    _check_qkv(q, k, v)
    B, H, N, D = q.shape
    q, qp = _f32(q)
    k, kp = _f32(k)
    v, vp = _f32(v)
    o = np.empty((B, H, N, D), np.float32)
    lse = np.empty((B, H, N), np.float32)
    fpp = ctypes.POINTER(ctypes.c_float)
    rc = lib().oracle_kernel_numerics(qp, kp, vp, o.ctypes.data_as(fpp), lse.ctypes.data_as(fpp),
                                      B, H, N, D, float(scale), int(bool(causal)), int(dtype),
                                      int(block_n))
    if rc != 0:
        raise RuntimeError(f"oracle_kernel_numerics failed: {rc}")
    return o, lse


def kernel_numerics_rows(q, k, v, scale, causal, sel_bh, sel_row, dtype=F16, block_n=64):
    """kernel_numerics for selected rows (flattened head bh = b*H + h, query
    row i).  Returns (o [n_sel, D] f32, lse [n_sel] f32)."""
    _check_qkv(q, k, v)
    B, H, N, D = q.shape
    q, qp = _f32(q)
    k, kp = _f32(k)
    v, vp = _f32(v)
    sel_bh = np.ascontiguousarray(sel_bh, dtype=np.int32)
    sel_row = np.ascontiguousarray(sel_row, dtype=np.int32)
    n = sel_bh.size
    o = np.empty((n, D), np.float32)
    lse = np.empty((n,), np.float32)
    ip = ctypes.POINTER(ctypes.c_int32)
    fpp = ctypes.POINTER(ctypes.c_float)
    rc = lib().oracle_kernel_numerics_rows(qp, kp, vp, B, H, N, D, float(scale),
                                           int(bool(causal)), int(dtype), int(block_n),
                                           sel_bh.ctypes.data_as(ip), sel_row.ctypes.data_as(ip),
                                           n, o.ctypes.data_as(fpp), lse.ctypes.data_as(fpp))
    if rc != 0:
        raise RuntimeError(f"oracle_kernel_numerics_rows failed: {rc}")
    return o, lse


def _round(fn, x):
    x, xp = _f32(x)
    out = np.empty_like(x)
    bits = np.empty(x.shape, np.uint16)
    fn(xp, out.ctypes.data_as(ctypes.POINTER(ctypes.c_float)),
       bits.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)), x.size)
    return out, bits


def round_f16(x):
    """fp32 -> fp16 (round-to-nearest-even): returns (values as f32, uint16 bits)."""
    return _round(lib().oracle_round_f16, x)


def round_bf16(x):
    """fp32 -> bf16 (round-to-nearest-even): returns (values as f32, uint16 bits)."""
    return _round(lib().oracle_round_bf16, x)


def num_threads() -> int:
    return int(lib().oracle_num_threads())


def set_num_threads(n: int) -> None:
    lib().oracle_set_num_threads(int(n))
