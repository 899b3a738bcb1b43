"""Seeded random problems aimed at each work plan of the forward: plain
grids, bound-driven split-KV, and one-round causal grids (pair mode, or the
XCD placement table at exactly two q-tiles per CU).  Each case records the plan the library chose for this device and
checks the result on sampled rows against the fp64 oracle and the
reference-kernel emulator (2x bars as in test_gpu_parity.py for random
problems), and against the one-workgroup-per-q-tile result (split_kv=False)
within the split-KV bounds of test_gpu_split.py.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import abi_ctypes as A
from helpers import LSE_TOL, case_seed, err_stats, make_qkv, to_np32
from test_gpu_split import _vs_unsplit

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _note(msg):
    print(msg, flush=True)


def _draw(case):
    """(B, H, N, D, dtype, causal, qk_sigma) aimed at plan kind case % 4."""
    rng = np.random.default_rng(case_seed(2000 + case))
    kind = case % 4
    D = int(rng.choice([64, 128]))
    dtype = str(rng.choice(["fp16", "bf16"]))
    sigma = float(rng.choice([1.0, 1.0, 2.0, 3.0]))
    if kind == 0:  # plain: many heads, short rows
        B, H = int(rng.integers(2, 5)), int(rng.integers(8, 33))
        N, causal = int(rng.integers(100, 1200)), bool(rng.integers(0, 2))
    elif kind == 1:  # bound-driven split: few heads, long rows
        B, H = 1, int(rng.integers(1, 5))
        N, causal = int(rng.integers(1500, 6000)), bool(rng.integers(0, 2))
    else:  # one round of 4-wave workgroups: pair mode (or the XCD placement table)
        hpx = int(rng.integers(1, 5))
        nq = int(rng.integers(32 // hpx + 1, 64 // hpx + 1))
        N = int(rng.integers((nq - 1) * 128 + 1, nq * 128 + 1))
        B = int(rng.choice([1, 2])) if (8 * hpx) % 2 == 0 else 1
        H = 8 * hpx // B
        causal = True
        if kind == 3:
            dtype = "bf16"  # bf16 causal keeps 4-wave workgroups at any N
    return B, H, N, D, dtype, causal, sigma


@pytest.fixture(scope="module")
def lib():
    return A.load()


@pytest.mark.parametrize("case", range(24))
def test_random_plans_vs_oracle(fa, oracle, lib, case):
    import ctypes

    B, H, N, D, dtype, causal, sigma = _draw(case)
    cus = int(fa.device_info(0)["compute_units"])
    q, k, v = make_qkv(B, H, N, D, dtype, seed=case_seed(2100 + case), qk_sigma=sigma,
                       device=DEV)
    p = A.params_from_tensors(q, k, v, torch.empty_like(q), None, causal)
    pl = A.FaFwdPlan()
    assert lib.fa_fwd_plan(ctypes.byref(p), cus, ctypes.byref(pl)) == A.FA_OK
    kind = ("pair" if pl.key_halves == 2 else "table" if pl.xcd_heads
            else "split" if pl.n_items else "plain")
    _note(f"case {case}: {B}x{H}x{N}x{D} {dtype} causal={causal} sigma={sigma} plan={kind}")
    o, lse = fa.forward(q, k, v, causal=causal, return_lse=True)
    o1, lse1 = fa.forward(q, k, v, causal=causal, return_lse=True, split_kv=False)
    torch.cuda.synchronize()
    assert torch.isfinite(o).all().item()
    if kind in ("plain", "table", "pair"):
        assert torch.equal(o, o1) and torch.equal(lse, lse1)
    else:
        _vs_unsplit(o, lse, o1, lse1, dtype)
    rng = np.random.default_rng(2200 + case)
    rows = sorted(set([0, 1, N // 2, N - 1] + rng.integers(0, N, size=20).tolist()))
    bhs = sorted({0, B * H - 1, (B * H) // 2})
    sel_bh = np.array([b for b in bhs for _ in rows], np.int32)
    sel_row = np.array([r for _ in bhs for r in rows], np.int32)
    qn, kn, vn = (to_np32(t.reshape(1, B * H, N, D)) for t in (q, k, v))
    scale = 1.0 / math.sqrt(D)
    ref_o, ref_lse = oracle.attn_rows_f64(qn, kn, vn, scale, causal, sel_bh, sel_row)
    emu_o, _ = oracle.kernel_numerics_rows(qn, kn, vn, scale, causal, sel_bh, sel_row,
                                           oracle.BF16 if dtype == "bf16" else oracle.F16)
    got_o = to_np32(o.reshape(B * H, N, D))[sel_bh, sel_row]
    got_lse = to_np32(lse.reshape(B * H, N))[sel_bh, sel_row]
    mx, mean = err_stats(got_o, ref_o)
    emx, emean = err_stats(emu_o, ref_o)
    lse_err = float(np.abs(got_lse.astype(np.float64) - ref_lse).max())
    _note(f"  {len(sel_row)} rows: max_abs={mx:.3e} mean_abs={mean:.3e} "
          f"(ref-kernel emu {emx:.3e}/{emean:.3e}) lse={lse_err:.3e}")
    assert mx <= 2 * emx + 1e-6 and mean <= 2 * emean + 1e-6
    assert lse_err <= LSE_TOL
