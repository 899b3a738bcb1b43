"""Writes tests/golden/c1_golden.npz: the C1 configuration (1x2x128x64 fp16,
seed 1234 + 100003*0, the reference's input convention in
benchmark/python/input_data.py:11-30) with expected O and LSE.

The expected values come from the reference's own formula
softmax(Q K^T * scale) V (benchmark/python/tests/test_pybind_correctness.py:
23-27) evaluated in numpy float64 on the fp16-quantised inputs — an
implementation independent of oracle/attn_oracle.c — and are cross-checked
against torch.nn.functional.scaled_dot_product_attention in float64 before
being written.  Nothing from the reference repository is imported or run.

Usage: python tests/golden/make_golden.py
"""
from __future__ import annotations

import math
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def softmax_attention_f64(q, k, v, scale, causal):
    s = np.einsum("bhid,bhjd->bhij", q, k) * scale
    if causal:
        n = s.shape[-1]
        s = np.where(np.triu(np.ones((n, n), bool), 1), -np.inf, s)
    m = s.max(-1, keepdims=True)
    p = np.exp(s - m)
    l = p.sum(-1, keepdims=True)
    return (p / l) @ v, (m + np.log(l))[..., 0]


def main():
    B, H, N, D = 1, 2, 128, 64
    seed = 1234 + 100003 * 0
    g = torch.Generator().manual_seed(seed)
    q, k, v = (torch.randn((B, H, N, D), generator=g).to(torch.float16) for _ in range(3))
    scale = 1.0 / math.sqrt(D)
    qd, kd, vd = (t.double().numpy() for t in (q, k, v))
    out = {}
    for causal, suffix in ((False, ""), (True, "_causal")):
        o, lse = softmax_attention_f64(qd, kd, vd, scale, causal)
        ref = torch.nn.functional.scaled_dot_product_attention(
            *(torch.from_numpy(x) for x in (qd, kd, vd)), is_causal=causal, scale=scale)
        assert np.abs(o - ref.numpy()).max() < 1e-12
        out["o_ref" + suffix] = o
        out["lse_ref" + suffix] = lse
    np.savez_compressed(
        os.path.join(HERE, "c1_golden.npz"),
        q_f16=q.numpy().view(np.uint16), k_f16=k.numpy().view(np.uint16),
        v_f16=v.numpy().view(np.uint16), scale=np.float64(scale), causal=np.bool_(False),
        seed=np.int64(seed), **out)
    print("wrote", os.path.join(HERE, "c1_golden.npz"))


if __name__ == "__main__":
    main()
