"""Shared test helpers: the BASELINE configs, seeded inputs and error metrics.

Input generation mirrors the reference's `random` mode
(benchmark/python/input_data.py:11-30): seed = base + 100003 * case_index,
Q, K, V ~ N(0, 1) drawn with a seeded torch.Generator, then cast to the
compute dtype (round-to-nearest-even).  Config C5 scales Q and K by 3 before
the cast to stress the online-softmax rescaling.
"""
from __future__ import annotations

import math

import numpy as np
import torch

BASE_SEED = 1234  # benchmark_pybind.py:201 default --seed

# id: (B, H, N, D, dtype, causal, qk_sigma, case_index)
CONFIGS = {
    "C1": (1, 2, 128, 64, "fp16", False, 1.0, 0),
    "C2": (4, 16, 1024, 64, "fp16", False, 1.0, 1),
    "C3": (4, 32, 4096, 128, "fp16", False, 1.0, 2),
    "C4": (2, 32, 8192, 128, "bf16", True, 1.0, 3),
    "C5": (1, 16, 16384, 128, "fp16", True, 3.0, 4),
    "C5r": (1, 16, 3000, 128, "fp16", True, 3.0, 5),
}

TORCH_DTYPES = {"fp16": torch.float16, "bf16": torch.bfloat16}

# Tolerances from the north-star contract.
MAX_ABS_TOL = 1e-2
MEAN_ABS_TOL = 1e-3
LSE_TOL = 1e-3


def case_seed(case_index: int, base: int = BASE_SEED) -> int:
    """input_data.py:11-12."""
    return int(base + case_index * 100_003)


def make_qkv(B, H, N, D, dtype, *, seed, qk_sigma=1.0, device="cpu"):
    """Seeded Q, K, V [B, H, N, D] in `dtype` ("fp16"/"bf16")."""
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    shape = (B, H, N, D)
    td = TORCH_DTYPES[dtype]
    q = torch.randn(shape, generator=gen, device=device, dtype=torch.float32)
    k = torch.randn(shape, generator=gen, device=device, dtype=torch.float32)
    v = torch.randn(shape, generator=gen, device=device, dtype=torch.float32)
    if qk_sigma != 1.0:
        q = q * qk_sigma
        k = k * qk_sigma
    return q.to(td).contiguous(), k.to(td).contiguous(), v.to(td).contiguous()


def make_config(name, device="cpu"):
    B, H, N, D, dtype, causal, sigma, case = CONFIGS[name]
    q, k, v = make_qkv(B, H, N, D, dtype, seed=case_seed(case), qk_sigma=sigma, device=device)
    return q, k, v, causal, 1.0 / math.sqrt(D)


def to_np32(t: torch.Tensor) -> np.ndarray:
    return t.detach().to("cpu", torch.float32).contiguous().numpy()


def err_stats(out, ref):
    """max-abs and mean-abs error of out against ref (numpy arrays)."""
    d = np.abs(np.asarray(out, np.float64) - np.asarray(ref, np.float64))
    return float(d.max()) if d.size else 0.0, float(d.mean()) if d.size else 0.0


def attention_flops(B, H, N, D, causal):
    """BASELINE.json metric: 4*B*H*N^2*D, halved for causal."""
    f = 4.0 * B * H * N * N * D
    return f / 2 if causal else f
