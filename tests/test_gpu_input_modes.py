"""GPU parity on the reference's non-random input modes (structured and
stress, benchmark/python/input_data.py:33-60) against the fp64 oracle.

structured inputs are smooth with |O| up to ~1.2: the absolute contract
applies, except the 1e-3 mean bar for bf16 output, where rounding O to bf16
alone (ulp 2^-7 on [1, 2)) costs ~1.2e-3 on average — the emulated reference
kernel measures the same — so bf16 mean-abs is held to the 2x bar only.
stress inputs (Q, K ~ 32 N(0,1) with +-256 outliers, V ~ 16 N(0,1) with +64
outliers) put |O| near 100 and |LSE| in the thousands, where one fp16 ulp of
O is 0.06: the absolute 1e-2 bar cannot hold for any fp16 output, so stress
is held to the 2x-reference-kernel bar (emulated arithmetic of the reference
kernel against the same oracle) and LSE to fp32 relative accuracy.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from fa_bench.input_data import generate_qkv
from helpers import LSE_TOL, MAX_ABS_TOL, MEAN_ABS_TOL, err_stats, to_np32

pytestmark = pytest.mark.gpu


def _run(fa, oracle, mode, D, dtype, causal, N=520, H=3):
    td = torch.float16 if dtype == "fp16" else torch.bfloat16
    q, k, v, _ = generate_qkv(batch_size=1, n_heads=H, seq_len=N, d_head=D, dtype=td,
                              device="cpu", input_mode=mode, seed=1234, case_index=11)
    scale = 1.0 / math.sqrt(D)
    o, lse = fa.forward(q.cuda(), k.cuda(), v.cuda(), causal=causal, return_lse=True)
    torch.cuda.synchronize()
    qn, kn, vn = to_np32(q), to_np32(k), to_np32(v)
    ref_o, ref_lse = oracle.attn_f64(qn, kn, vn, scale, causal)
    emu_o, emu_lse = oracle.kernel_numerics(qn, kn, vn, scale, causal,
                                            oracle.BF16 if dtype == "bf16" else oracle.F16)
    mx, mean = err_stats(to_np32(o), ref_o)
    emx, emean = err_stats(emu_o, ref_o)
    lse_err = np.abs(to_np32(lse).astype(np.float64) - ref_lse)
    print(f"  max_abs={mx:.3e} mean_abs={mean:.3e} (emu {emx:.3e}/{emean:.3e}) "
          f"lse_err={lse_err.max():.3e} |lse|max={np.abs(ref_lse).max():.1f}", flush=True)
    assert np.isfinite(to_np32(o)).all()
    return mx, mean, emx, emean, lse_err, ref_lse


@pytest.mark.parametrize("causal", [False, True], ids=["noncausal", "causal"])
@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("D", [64, 128])
def test_structured_inputs(fa, oracle, D, dtype, causal):
    print(f"case structured D={D} {dtype} causal={causal}", flush=True)
    mx, mean, emx, emean, lse_err, _ = _run(fa, oracle, "structured", D, dtype, causal)
    assert mx <= MAX_ABS_TOL
    if dtype == "fp16":
        assert mean <= MEAN_ABS_TOL
    assert mx <= 2 * emx + 1e-6 and mean <= 2 * emean + 1e-6
    assert lse_err.max() <= LSE_TOL


@pytest.mark.parametrize("causal", [False, True], ids=["noncausal", "causal"])
@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("D", [64, 128])
def test_stress_inputs(fa, oracle, D, dtype, causal):
    print(f"case stress D={D} {dtype} causal={causal}", flush=True)
    mx, mean, emx, emean, lse_err, ref_lse = _run(fa, oracle, "stress", D, dtype, causal)
    assert mx <= 2 * emx + 1e-6, f"max-abs {mx} > 2x reference-kernel error {emx}"
    assert mean <= 2 * emean + 1e-6, f"mean-abs {mean} > 2x reference-kernel error {emean}"
    # fp32 scores of magnitude ~1e4: LSE to a few fp32 ulps of |LSE|
    assert (lse_err <= LSE_TOL + 4e-6 * np.abs(ref_lse)).all()
