"""Closed-form and invariance checks that pin an attention implementation
without trusting any other implementation.

`pin_failures(attn)` runs every check on `attn(q, k, v, scale, causal) ->
(o, lse)` (float64 numpy outputs) and returns the names of the failing checks.
The checks are chosen so that each plausible mistake (dropped scale, causal
off-by-one, LSE missing the max, transposed scores, missing normalisation)
fails at least one of them; tests/test_oracle.py proves that by planting each
mistake in the oracle.
"""
from __future__ import annotations

import math

import numpy as np


def _rand(rng, shape, scale=1.0):
    # values exactly representable in fp16 (and float32): multiples of 2^-8
    return (np.round(rng.standard_normal(shape) * scale * 256.0) / 256.0).astype(np.float32)


def pin_failures(attn, tol=1e-9):
    rng = np.random.default_rng(20240601)
    fails = []

    def close(a, b, t=tol):
        return np.allclose(np.asarray(a, np.float64), np.asarray(b, np.float64), atol=t, rtol=0)

    for causal in (False, True):
        B, H, N, D = 1, 2, 37, 16
        k = _rand(rng, (B, H, N, D))
        v = _rand(rng, (B, H, N, D))
        q = _rand(rng, (B, H, N, D))
        scale = 1.0 / math.sqrt(D)
        tag = "causal" if causal else "full"

        # 1. Q = 0: every visible score is 0 -> O_i = mean of visible V, LSE_i = ln(#visible)
        o, lse = attn(np.zeros_like(q), k, v, scale, causal)
        cnt = np.arange(1, N + 1, dtype=np.float64) if causal else np.full(N, float(N))
        if causal:
            ref = np.cumsum(v.astype(np.float64), axis=2) / cnt[None, None, :, None]
        else:
            ref = np.broadcast_to(v.astype(np.float64).mean(axis=2, keepdims=True), v.shape)
        if not close(o, ref):
            fails.append(f"zero_q_mean_{tag}")
        if not close(lse, np.broadcast_to(np.log(cnt), lse.shape)):
            fails.append(f"zero_q_lse_{tag}")

        # 2. V constant -> O constant
        vc = np.full_like(v, 0.75)
        o, _ = attn(q, k, vc, scale, causal)
        if not close(o, 0.75):
            fails.append(f"const_v_{tag}")

        # 3. N = 1 -> O = V_0, LSE = scale * q.k
        o, lse = attn(q[:, :, :1], k[:, :, :1], v[:, :, :1], scale, causal)
        if not close(o, v[:, :, :1]):
            fails.append(f"n1_output_{tag}")
        qk = (q[:, :, 0].astype(np.float64) * k[:, :, 0].astype(np.float64)).sum(-1) * scale
        if not close(lse[:, :, 0], qk):
            fails.append(f"n1_lse_{tag}")

        # 4. Scale enters only through scale * Q.K: O(q, s) == O(s' q, s / s') with s' = 2
        o1, l1 = attn(q, k, v, scale, causal)
        o2, l2 = attn(q * 2.0, k, v, scale / 2.0, causal)
        if not (close(o1, o2, 1e-12) and close(l1, l2, 1e-12)):
            fails.append(f"scale_folding_{tag}")
        o3, _ = attn(q, k, v, scale * 3.0, causal)
        if close(o1, o3, 1e-6):
            fails.append(f"scale_ignored_{tag}")

        # 5. Adding w to every key shifts row i's scores by scale * q_i.w:
        #    O unchanged, LSE shifted by that amount.
        w = np.round(rng.standard_normal(D) * 4.0).astype(np.float32)  # small integers
        o4, l4 = attn(q, k + w, v, scale, causal)
        shift = scale * (q.astype(np.float64) @ w.astype(np.float64))
        if not close(o4, o1, 1e-9):
            fails.append(f"key_shift_output_{tag}")
        if not close(l4, l1 + shift, 1e-9):
            fails.append(f"key_shift_lse_{tag}")

        # 6. Linearity in V
        v2 = _rand(rng, v.shape)
        oa, _ = attn(q, k, v, scale, causal)
        ob, _ = attn(q, k, v2, scale, causal)
        oc, _ = attn(q, k, v + v2, scale, causal)
        if not close(oc, oa + ob, 1e-9):
            fails.append(f"linear_v_{tag}")

        # 7. Causal row 0 sees only key 0; last row sees every key (= non-causal)
        if causal:
            of, lf = attn(q, k, v, scale, False)
            if not close(o1[:, :, 0], v[:, :, 0]):
                fails.append("causal_row0")
            if not (close(o1[:, :, -1], of[:, :, -1]) and close(l1[:, :, -1], lf[:, :, -1])):
                fails.append("causal_last_row")

    # 8. Non-causal key permutation invariance
    B, H, N, D = 1, 1, 29, 8
    q = _rand(rng, (B, H, N, D))
    k = _rand(rng, (B, H, N, D))
    v = _rand(rng, (B, H, N, D))
    perm = rng.permutation(N)
    o1, l1 = attn(q, k, v, 0.5, False)
    o2, l2 = attn(q, k[:, :, perm], v[:, :, perm], 0.5, False)
    if not (close(o1, o2, 1e-12) and close(l1, l2, 1e-12)):
        fails.append("key_permutation")
    # 9. One dominant key: q_i = t * k_0 direction with large t -> O_i ~= V_0
    k = _rand(rng, (B, H, N, D))
    q = np.broadcast_to(k[:, :, :1] * 64.0, (B, H, N, D)).astype(np.float32)
    kd = k.copy()
    kd[:, :, 1:] *= 0.01
    o, _ = attn(q, kd, v, 1.0, False)
    if not close(o, np.broadcast_to(v[:, :, :1], o.shape), 1e-6):
        fails.append("dominant_key")
    return fails
