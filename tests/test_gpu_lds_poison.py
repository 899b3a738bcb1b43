"""GPU runs of the LDS-poison debug build (libfa_mi355x_poison.so: the kernel
source compiled with -DFA_LDS_POISON, same ABI).

In that build every wave fills the LDS bytes it is about to stage (K/V ring
slots before their DMA, staged Q, the output rows, the pair-mode combine
area) with all-ones words, NaN in fp16, bf16 and fp32, and waits for the
fill before the staging write.  A read that ran ahead of its wait or barrier
would pick up NaN instead of the previous tile's plausible values.  With
correct synchronisation the output must equal the product build's bit for
bit, which each case checks for O and the LSE, on the plain grid (fa_fwd)
and with a workspace (fa_fwd_ws, where the plan may split).

Shapes: one and two key tiles (N = 64, 128), ragged tails, causal
diagonals, 4- and 8-wave workgroups, pair mode, split-KV with its merge, the
XCD placement table, fp16 and bf16, D = 64 and 128, and Q, K ~ N(0, 3^2)
inputs whose offsets are re-derived mid-row.
"""
from __future__ import annotations

import ctypes
import os

import pytest
import torch

import abi_ctypes as A
from helpers import case_seed, make_qkv

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module")
def libs():
    if not os.path.exists(A.POISON_LIB_PATH):
        pytest.fail("libfa_mi355x_poison.so is missing: run build() first")
    return A.load(A.LIB_PATH), A.load(A.POISON_LIB_PATH)


def _run(L, q, k, v, causal, use_ws):
    o = torch.full_like(q, float("nan"))
    lse = torch.full(q.shape[:3], float("nan"), dtype=torch.float32, device=DEV)
    p = A.params_from_tensors(q, k, v, o, lse=lse, causal=causal)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    if use_ws:
        need = ctypes.c_uint64(0)
        assert L.fa_fwd_workspace_size(ctypes.byref(p), ctypes.byref(need)) == A.FA_OK
        ws = torch.empty(max(int(need.value), 16), dtype=torch.uint8, device=DEV)
        rc = L.fa_fwd_ws(ctypes.byref(p), ctypes.c_void_p(ws.data_ptr()), need.value, stream)
    else:
        rc = L.fa_fwd(ctypes.byref(p), stream)
    assert rc == A.FA_OK, L.fa_last_error()
    torch.cuda.synchronize()
    return o, lse


CASES = [
    # B, H, N, D, dtype, causal, Q/K scale
    (1, 2, 64, 64, "fp16", False, 1.0),     # one key tile
    (1, 2, 128, 128, "fp16", False, 1.0),   # two key tiles
    (1, 2, 64, 128, "bf16", True, 1.0),
    (1, 2, 128, 64, "bf16", True, 1.0),
    (1, 3, 100, 128, "fp16", True, 1.0),    # ragged tail on the diagonal
    (2, 2, 1000, 64, "bf16", False, 1.0),
    (1, 2, 2304, 128, "fp16", False, 1.0),  # 8-wave workgroups (optimistic pass)
    (1, 2, 2100, 64, "bf16", False, 3.0),   # 8-wave checked pass, re-derivations
    (1, 1, 8192, 128, "fp16", True, 1.0),   # 8-wave causal
    (1, 8, 3000, 128, "fp16", True, 3.0),   # pair mode
    (1, 8, 3000, 64, "bf16", True, 1.0),
    (1, 16, 4096, 128, "fp16", True, 1.0),  # XCD placement table (256 CUs)
    (1, 4, 3000, 128, "fp16", True, 3.0),   # split-KV with a workspace
]


@pytest.mark.parametrize("use_ws", [False, True], ids=["plain", "workspace"])
@pytest.mark.parametrize("B,H,N,D,dtype,causal,sig", CASES)
def test_poison_build_matches_product_bitwise(libs, B, H, N, D, dtype, causal, sig, use_ws):
    print(f"case poison B={B} H={H} N={N} D={D} {dtype} causal={causal} sig={sig} "
          f"ws={use_ws}", flush=True)
    prod, poison = libs
    q, k, v = make_qkv(B, H, N, D, dtype, seed=case_seed(B * 7919 + H * 131 + N + D),
                       qk_sigma=sig, device="cpu")
    q, k, v = q.to(DEV), k.to(DEV), v.to(DEV)
    o_ref, lse_ref = _run(prod, q, k, v, causal, use_ws)
    o, lse = _run(poison, q, k, v, causal, use_ws)
    assert torch.isfinite(o).all() and torch.isfinite(lse).all()
    assert torch.equal(o.view(torch.int16), o_ref.view(torch.int16))
    assert torch.equal(lse.view(torch.int32), lse_ref.view(torch.int32))
