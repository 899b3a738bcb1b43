"""GPU parity of both MFMA forms of the fp16 8-wave non-causal kernel: the
product's 16x16x32 kernel (csrc/fa_fwd16.inc, libfa_mi355x.so) and the
32x32x16 form of fa_fwd_kernel (libfa_mi355x_mfma32.so: the kernel source
compiled with -DFA_MFMA32, same ABI), which exists to compare the two
shapes by counters (profiles/mfma_shape_16x16_vs_32x32.md); its results must
meet the same bars as the product's before its counters mean anything.

Each case runs through the C ABI (fa_fwd) and checks every element of O and
the LSE against the fp64 oracle and the reference-kernel emulator, at the
contract bars for N(0, 1) inputs and at the non-contract bars for the
Q, K ~ N(0, 3^2) inputs that send the kernel to its second (plain online
softmax) pass.  It also checks that the product library, fed the same
inputs, stays within two output roundings of it: the two forms sum S in a
different order, so they agree to rounding, not bit for bit.
"""
from __future__ import annotations

import ctypes
import math
import os

import pytest
import torch

import abi_ctypes as A
from helpers import case_seed, make_qkv
from test_gpu_parity import _check_against_oracle

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module")
def libs():
    if not os.path.exists(A.MFMA32_LIB_PATH):
        pytest.fail("libfa_mi355x_mfma32.so is missing: run build() first")
    return A.load(A.LIB_PATH), A.load(A.MFMA32_LIB_PATH)


def _run(L, q, k, v):
    o = torch.full_like(q, float("nan"))
    lse = torch.full(q.shape[:3], float("nan"), dtype=torch.float32, device=DEV)
    p = A.params_from_tensors(q, k, v, o, lse=lse, causal=False)
    rc = L.fa_fwd(ctypes.byref(p), ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == A.FA_OK, L.fa_last_error()
    torch.cuda.synchronize()
    return o, lse


@pytest.mark.parametrize("B,H,N,sigma", [
    (1, 2, 2048, 1.0),   # 32 key tiles, optimistic pass
    (1, 2, 2049, 1.0),   # ragged last tile (one key)
    (1, 3, 2300, 1.0),   # ragged, 9 q-tiles of 256 rows
    (2, 2, 4096, 1.0),   # C3's row length
    (1, 2, 2112, 3.0),   # wide scores: the spread test sends it to the second pass
])
def test_mfma_shapes_vs_oracle(libs, oracle, B, H, N, sigma):
    prod, mfma32 = libs
    print(f"case mfma shapes B={B} H={H} N={N} sigma={sigma}", flush=True)
    q, k, v = make_qkv(B, H, N, 128, "fp16", seed=case_seed(1600 + N), qk_sigma=sigma, device=DEV)
    scale = 1.0 / math.sqrt(128)
    o, lse = _run(prod, q, k, v)
    _check_against_oracle(oracle, q, k, v, o, lse, False, scale, "fp16", contract=sigma == 1.0)
    o1, lse1 = _run(mfma32, q, k, v)
    _check_against_oracle(oracle, q, k, v, o1, lse1, False, scale, "fp16", contract=sigma == 1.0)
    d = (o.float() - o1.float()).abs()
    bound = 2.0 ** -9 * (1.0 + o1.float().abs())
    print(f"  16x16x32 vs 32x32x16: max|dO|={d.max().item():.3e} "
          f"max|dLSE|={(lse - lse1).abs().max().item():.3e}", flush=True)
    assert bool((d <= bound).all())
    assert (lse - lse1).abs().max().item() <= 2.0 ** -10 + 1e-5
