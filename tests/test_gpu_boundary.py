"""The drop-in boundary on the GPU.

- The torch extension's `forward(q, k, v, o, benchmark)` keeps the
  reference's result: a pair `(o, ms)` that the reference wrapper indexes and
  unpacks (python/flash_attention_runtime/__init__.py:31,37; the extension
  python/flash_attention_runtime/_ext.cu:124-158,162-172).  The extensions are
  keyword-only, and only `return_lse=True` adds a third element.
- The C ABI reports its own launch status: a HIP error that the caller's
  thread left behind before `fa_fwd` is neither reported by `fa_fwd` nor
  cleared by it.
"""
from __future__ import annotations

import ctypes
import ctypes.util
import math

import pytest
import torch

import abi_ctypes as A
from helpers import make_qkv, case_seed

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _note(msg):
    print(msg, flush=True)


def test_extension_result_unpacks_like_the_reference(fa):
    _note("case extension (o, ms) contract")
    ext = fa._EXT
    q, k, v = make_qkv(1, 2, 256, 128, "fp16", seed=case_seed(31), device=DEV)
    o = torch.empty_like(q)
    # python/flash_attention_runtime/__init__.py:31
    out = ext.forward(q, k, v, o, False)[0]
    assert out.data_ptr() == o.data_ptr()
    res = ext.forward(q, k, v, None, False)
    assert isinstance(res, tuple) and len(res) == 2
    assert torch.equal(res[0], out) and res[1] == 0.0
    # python/flash_attention_runtime/__init__.py:37
    out2, runtime_ms = ext.forward(q, k, v, o, True)
    assert isinstance(runtime_ms, float) and runtime_ms > 0.0
    assert torch.equal(out2, out)
    # keyword arguments and the defaults of the reference
    out3, ms3 = ext.forward(q=q, k=k, v=v)
    assert torch.equal(out3, out) and ms3 == 0.0
    # the extensions are keyword-only; return_lse adds the LSE as a third element
    o4, ms4, lse = ext.forward(q, k, v, None, False, return_lse=True)
    assert torch.equal(o4, out) and lse.shape == (1, 2, 256) and lse.dtype == torch.float32
    with pytest.raises(TypeError):
        ext.forward(q, k, v, None, False, True)  # causal only by keyword
    # the package's own wrappers on top of it
    assert torch.equal(fa.forward(q, k, v), out)
    o5, ms5 = fa.forward_timed(q, k, v)
    assert torch.equal(o5, out) and ms5 > 0.0
    o6, ms6, lse6 = fa.forward_timed(q, k, v, return_lse=True)
    assert torch.equal(o6, out) and torch.equal(lse6, lse)


def _hip():
    name = ctypes.util.find_library("amdhip64") or "libamdhip64.so"
    h = ctypes.CDLL(name)
    for f in ("hipSetDevice", "hipGetLastError", "hipPeekAtLastError", "hipDeviceSynchronize"):
        getattr(h, f).restype = ctypes.c_int
    h.hipSetDevice.argtypes = [ctypes.c_int]
    return h


def test_stale_caller_error_is_neither_reported_nor_cleared(fa):
    """The caller's thread holds a failed HIP call (hipSetDevice of an invalid
    ordinal) when it calls fa_fwd: the launch succeeds, fa_fwd returns FA_OK
    with the correct output, and the caller's error is still there for the
    caller to read, as far as HIP itself keeps it across a successful call."""
    _note("case stale HIP error before fa_fwd")
    lib = A.load()
    hip = _hip()
    q, k, v = make_qkv(1, 2, 300, 64, "fp16", seed=case_seed(32), device=DEV)
    ref = fa.forward(q, k, v)
    o = torch.zeros_like(q)
    p = A.params_from_tensors(q, k, v, o)
    torch.cuda.synchronize()
    try:
        # Control: does HIP keep a thread's last error across a successful call?
        bad = hip.hipSetDevice(1 << 20)
        assert bad != 0
        assert hip.hipDeviceSynchronize() == 0
        hip_keeps_it = hip.hipPeekAtLastError() == bad
        hip.hipGetLastError()
        assert hip.hipPeekAtLastError() == 0

        assert hip.hipSetDevice(1 << 20) == bad
        st = lib.fa_fwd(ctypes.byref(p), None)
        assert st == A.FA_OK, lib.fa_last_error()
        assert lib.fa_last_error() == b""
        after = hip.hipPeekAtLastError()
        _note(f"  HIP keeps a stale error across a successful call: {hip_keeps_it}; "
              f"after fa_fwd: {after}")
        if hip_keeps_it:
            assert after == bad, "fa_fwd consumed the caller's pending HIP error"
        assert hip.hipDeviceSynchronize() == 0
    finally:
        hip.hipGetLastError()  # leave no error behind for torch's own checks
    assert torch.equal(o, ref)


def test_fa_fwd_timed_with_stale_error(fa):
    _note("case stale HIP error before fa_fwd_timed")
    lib = A.load()
    hip = _hip()
    q, k, v = make_qkv(1, 1, 130, 128, "bf16", seed=case_seed(33), device=DEV)
    ref = fa.forward(q, k, v, causal=True)
    o = torch.zeros_like(q)
    p = A.params_from_tensors(q, k, v, o, causal=True)
    torch.cuda.synchronize()
    ms = ctypes.c_float(-1.0)
    try:
        assert hip.hipSetDevice(1 << 20) != 0
        assert lib.fa_fwd_timed(ctypes.byref(p), None, ctypes.byref(ms)) == A.FA_OK
    finally:
        hip.hipGetLastError()
    assert ms.value > 0.0 and not math.isnan(ms.value)
    assert torch.equal(o, ref)
