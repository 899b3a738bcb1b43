"""GPU timing guards for data-dependent slow paths of the forward kernel.

The fp16 kernels with matrix-core row sums run an optimistic pass that
keeps the first key tile's row max as the exponent offset.  Inputs whose
scores spread widely (Q, K ~ N(0, 3^2), as the BASELINE causal config at
N = 16384 uses) would overflow it and force a recomputation of the whole
workgroup; the kernel instead leaves the optimistic pass after the first
tile.  A regression there doubles the time on such inputs while every
parity test still passes, so it is guarded here by timing: wide-score
inputs may cost a little more than N(0, 1) inputs (the checked pass), never
close to twice as much.  Both timings come from the same box in the same
process, so the bar (1.5x; measured 1.03-1.07x, the regression it guards
against 1.9x) does not depend on which MI355X runs it.
"""
from __future__ import annotations

import pytest
import torch

from helpers import case_seed, make_qkv

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _time(fa, q, k, v, causal, steps=20, warmup=5):
    o = torch.empty_like(q)
    for _ in range(warmup):
        fa.forward(q, k, v, o, causal=causal)
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(steps):
        fa.forward(q, k, v, o, causal=causal)
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / steps


@pytest.mark.parametrize("sigma", [1.5, 2.0, 3.0])
@pytest.mark.parametrize("causal,N", [(True, 8192), (False, 4096)],
                         ids=["causal8192", "noncausal4096"])
def test_wide_scores_do_not_double_the_time(fa, causal, N, sigma):
    """sigma 1.5 stays in the optimistic pass, 2 and 3 leave it after the
    first tile: neither may fall into a full recomputation."""
    B, H, D = 1, 16, 128
    print(f"case perf guard causal={causal} N={N} sigma={sigma}", flush=True)
    q1, k1, v1 = make_qkv(B, H, N, D, "fp16", seed=case_seed(950), device=DEV)
    q3, k3, v3 = make_qkv(B, H, N, D, "fp16", seed=case_seed(950), qk_sigma=sigma, device=DEV)
    t1 = min(_time(fa, q1, k1, v1, causal) for _ in range(2))
    t3 = min(_time(fa, q3, k3, v3, causal) for _ in range(2))
    print(f"  N(0,1): {t1:.4f} ms   N(0,{sigma}^2): {t3:.4f} ms   ratio {t3 / t1:.3f}",
          flush=True)
    assert t3 / t1 < 1.5
