"""fa_fwd_scratch, the entry point that allocates nothing: fa_fwd_ws with the
library's static per-device scratch array as the split-KV workspace.

Checked through the C ABI against fa_fwd_ws with a workspace from torch's
allocator (same plan, same kernels: bit for bit), on two calls in a row, the
second with a smaller problem; the device's free memory does not move across
a call; a problem whose split needs more than FA_SCRATCH_BYTES is rejected
before anything is launched; and a problem that needs no workspace gives
fa_fwd's result.
"""
from __future__ import annotations

import ctypes

import pytest
import torch

import abi_ctypes as A
from helpers import case_seed, make_qkv

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _note(msg):
    print(msg, flush=True)


def _problem(B, H, N, D, dtype, causal, sigma, seed):
    q, k, v = make_qkv(B, H, N, D, dtype, seed=case_seed(seed), qk_sigma=sigma, device=DEV)
    return q, k, v


def _outputs(q):
    o = torch.full_like(q, float("nan"))
    lse = torch.full(q.shape[:3], float("nan"), device=DEV, dtype=torch.float32)
    return o, lse


def _need(lib, p):
    need = ctypes.c_uint64(0)
    assert lib.fa_fwd_workspace_size(ctypes.byref(p), ctypes.byref(need)) == A.FA_OK
    return need.value


# (B, H, N, D, dtype, causal, qk_sigma): the first is C5r's shape and inputs
# with 4 of its 16 heads (bound-driven split of the long q-tiles), the second
# a smaller split.
SPLIT_CASES = [(1, 4, 3000, 128, "fp16", True, 3.0), (1, 1, 4096, 64, "bf16", False, 1.0)]


def test_scratch_matches_workspace_entry_two_calls():
    lib = A.load()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    sizes = []
    for i, (B, H, N, D, dtype, causal, sigma) in enumerate(SPLIT_CASES):
        _note(f"case scratch call {i + 1}: {B}x{H}x{N}x{D} {dtype} causal={causal}")
        q, k, v = _problem(B, H, N, D, dtype, causal, sigma, 4100 + i)
        o_ref, lse_ref = _outputs(q)
        p_ref = A.params_from_tensors(q, k, v, o_ref, lse_ref, causal)
        need = _need(lib, p_ref)
        assert 0 < need <= A.FA_SCRATCH_BYTES, need  # the plan really splits
        sizes.append(need)
        ws = torch.empty(need, dtype=torch.uint8, device=DEV)
        assert lib.fa_fwd_ws(ctypes.byref(p_ref), ctypes.c_void_p(ws.data_ptr()), need,
                             stream) == A.FA_OK
        o, lse = _outputs(q)
        p = A.params_from_tensors(q, k, v, o, lse, causal)
        torch.cuda.synchronize()
        free0, _ = torch.cuda.mem_get_info()
        st = lib.fa_fwd_scratch(ctypes.byref(p), stream)
        assert st == A.FA_OK, lib.fa_last_error()
        torch.cuda.synchronize()
        free1, _ = torch.cuda.mem_get_info()
        # fa_fwd_ws above already loaded the library's code object (and with
        # it the static scratch array) on this device, so every call counts.
        assert free1 == free0, (free0, free1)
        assert torch.equal(o, o_ref), "O differs from fa_fwd_ws"
        assert torch.equal(lse, lse_ref), "LSE differs from fa_fwd_ws"
    assert sizes[1] < sizes[0]


def test_scratch_rejects_a_plan_beyond_its_size():
    lib = A.load()
    B, H, N, D = 1, 5, 6000, 128  # non-causal split of 46 MiB on 256 CUs
    _note(f"case scratch too small: {B}x{H}x{N}x{D}")
    q, k, v = _problem(B, H, N, D, "fp16", False, 1.0, 4200)
    o, lse = _outputs(q)
    p = A.params_from_tensors(q, k, v, o, lse, False)
    need = _need(lib, p)
    if need <= A.FA_SCRATCH_BYTES:
        pytest.skip(f"this device's plan needs only {need} bytes")
    assert lib.fa_fwd_scratch(ctypes.byref(p), None) == A.FA_ERR_UNSUPPORTED
    assert b"static scratch" in lib.fa_last_error()
    torch.cuda.synchronize()
    assert torch.isnan(o).all().item() and torch.isnan(lse).all().item()


@pytest.mark.parametrize("B,H,N,causal", [(2, 8, 700, False), (1, 8, 3000, True)],
                         ids=["plain", "pair-mode"])
def test_scratch_unsplit_problem_equals_fa_fwd(B, H, N, causal):
    lib = A.load()
    _note(f"case scratch with an unsplit problem {B}x{H}x{N} causal={causal}")
    q, k, v = _problem(B, H, N, 128, "fp16", causal, 1.0, 4300)
    o_ref, lse_ref = _outputs(q)
    p_ref = A.params_from_tensors(q, k, v, o_ref, lse_ref, causal)
    assert _need(lib, p_ref) == 0
    assert lib.fa_fwd(ctypes.byref(p_ref), None) == A.FA_OK
    o, lse = _outputs(q)
    p = A.params_from_tensors(q, k, v, o, lse, causal)
    assert lib.fa_fwd_scratch(ctypes.byref(p), None) == A.FA_OK
    torch.cuda.synchronize()
    assert torch.equal(o, o_ref) and torch.equal(lse, lse_ref)
