"""CPU tests that pin the oracle (oracle/attn_oracle.c) before it is trusted
as the GPU checker.

Pins, in order of independence from the oracle's own code:
  * the committed golden fixture for config C1 (expected O/LSE computed by
    tests/golden/make_golden.py with the reference's matrix formula
    softmax(Q K^T * scale) V — test_pybind_correctness.py:23-27 — in numpy
    float64, cross-checked there against torch's CPU SDPA);
  * torch.nn.functional.scaled_dot_product_attention in float64 (a library
    routine) on random shapes, causal and not;
  * closed forms and invariances (tests/oracle_pins.py), which every planted
    mistake must fail (mutation tests below).
The reference ships no golden vectors of its own (benchmark/data/replay holds
only .gitkeep); its MMA known-answer tests are re-derived for MFMA in
tests/test_gpu_kat.py.
"""
from __future__ import annotations

import math
import os

import numpy as np
import pytest
import torch

from oracle_pins import pin_failures

HERE = os.path.dirname(os.path.abspath(__file__))


def _attn(oracle, mutation=0):
    def f(q, k, v, scale, causal):
        return oracle.attn_f64(q, k, v, scale, causal, mutation)

    return f


def _rand_inputs(shape, seed, dtype="fp16"):
    g = torch.Generator().manual_seed(seed)
    td = torch.float16 if dtype == "fp16" else torch.bfloat16
    return [torch.randn(shape, generator=g).to(td).float().numpy() for _ in range(3)]


def test_oracle_passes_all_pins(oracle):
    assert pin_failures(_attn(oracle)) == []


@pytest.mark.parametrize("mutation", ["no_scale", "causal_diag", "lse_no_max", "transpose_s",
                                      "no_normalise"])
def test_planted_mistake_is_caught(oracle, mutation):
    """Each plausible oracle mistake fails at least one closed-form check."""
    fails = pin_failures(_attn(oracle, oracle.MUTATIONS[mutation]))
    assert fails, f"mutation {mutation} passed every pin"


def test_golden_c1_fixture(oracle):
    path = os.path.join(HERE, "golden", "c1_golden.npz")
    z = np.load(path)  # allow_pickle=False (default)
    q = z["q_f16"].view(np.float16).astype(np.float32)
    k = z["k_f16"].view(np.float16).astype(np.float32)
    v = z["v_f16"].view(np.float16).astype(np.float32)
    o, lse = oracle.attn_f64(q, k, v, float(z["scale"]), bool(z["causal"]))
    assert np.abs(o - z["o_ref"]).max() <= 1e-12
    assert np.abs(lse - z["lse_ref"]).max() <= 1e-12
    oc, lc = oracle.attn_f64(q, k, v, float(z["scale"]), True)
    assert np.abs(oc - z["o_ref_causal"]).max() <= 1e-12
    assert np.abs(lc - z["lse_ref_causal"]).max() <= 1e-12


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("N,D", [(1, 64), (7, 64), (65, 128), (130, 64), (200, 128)])
def test_oracle_vs_torch_sdpa_f64(oracle, N, D, causal):
    q, k, v = _rand_inputs((2, 3, N, D), seed=N * 31 + D)
    scale = 1.0 / math.sqrt(D)
    o, lse = oracle.attn_f64(q, k, v, scale, causal)
    tq, tk, tv = (torch.from_numpy(x).double() for x in (q, k, v))
    ref = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, is_causal=causal,
                                                           scale=scale)
    s = (tq @ tk.transpose(-1, -2)) * scale
    if causal:
        s = s.masked_fill(torch.ones(N, N, dtype=torch.bool).triu(1), float("-inf"))
    ref_lse = torch.logsumexp(s, dim=-1)
    assert np.abs(o - ref.numpy()).max() <= 1e-10
    assert np.abs(lse - ref_lse.numpy()).max() <= 1e-10


def test_rows_api_matches_full(oracle):
    q, k, v = _rand_inputs((2, 2, 90, 64), seed=5)
    o, lse = oracle.attn_f64(q, k, v, 0.125, True)
    sel_bh = np.array([0, 3, 1, 2], np.int32)
    sel_row = np.array([0, 89, 45, 64], np.int32)
    os_, ls = oracle.attn_rows_f64(q, k, v, 0.125, True, sel_bh, sel_row)
    of = o.reshape(4, 90, 64)
    lf = lse.reshape(4, 90)
    assert np.array_equal(os_, of[sel_bh, sel_row])
    assert np.array_equal(ls, lf[sel_bh, sel_row])


@pytest.mark.parametrize("causal", [False, True])
def test_reference_cpu_path_restatement(oracle, causal):
    """oracle_ref_online_f32 (the reference CPU path, correctness_v6.cu:23-72)
    agrees with the exact oracle to fp32 accuracy."""
    q, k, v = _rand_inputs((1, 2, 128, 64), seed=11)
    o, _ = oracle.attn_f64(q, k, v, 0.125, causal)
    o32 = oracle.ref_online_f32(q, k, v, 0.125, causal)
    assert np.abs(o32 - o).max() <= 2e-5
    part = oracle.ref_online_f32(q, k, v, 0.125, causal, row_begin=10, row_end=20)
    flat = part.reshape(-1, 64)
    assert np.isnan(flat[:10]).all() and np.isnan(flat[20:]).all()
    assert np.array_equal(flat[10:20], o32.reshape(-1, 64)[10:20])


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("causal", [False, True])
def test_kernel_numerics_emulator(oracle, dtype, causal):
    """The reference-kernel emulator is within the contract tolerance of the
    exact oracle, but not identical to it (it really rounds P and O)."""
    q, k, v = _rand_inputs((1, 2, 300, 128), seed=3, dtype=dtype)
    o, lse = oracle.attn_f64(q, k, v, 1 / math.sqrt(128), causal)
    eo, el = oracle.kernel_numerics(q, k, v, 1 / math.sqrt(128), causal,
                                    oracle.BF16 if dtype == "bf16" else oracle.F16)
    d = np.abs(eo - o)
    assert d.max() <= 1e-2 and d.mean() <= 1e-3
    assert d.max() > 0
    assert np.abs(el - lse).max() <= 1e-4


@pytest.mark.parametrize("causal", [False, True])
def test_kernel_numerics_rows_matches_full(oracle, causal):
    """The row-selective emulator is the full emulator restricted to the
    selected rows, bit for bit."""
    q, k, v = _rand_inputs((2, 2, 150, 64), seed=9)
    eo, el = oracle.kernel_numerics(q, k, v, 0.125, causal, oracle.F16)
    sel_bh = np.array([0, 3, 1, 2, 3], np.int32)
    sel_row = np.array([0, 149, 64, 63, 100], np.int32)
    ro, rl = oracle.kernel_numerics_rows(q, k, v, 0.125, causal, sel_bh, sel_row, oracle.F16)
    assert np.array_equal(ro, eo.reshape(4, 150, 64)[sel_bh, sel_row])
    assert np.array_equal(rl, el.reshape(4, 150)[sel_bh, sel_row])


def test_round_f16_matches_numpy(oracle):
    rng = np.random.default_rng(0)
    x = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * 10,
        rng.standard_normal(50000).astype(np.float32) * 1e-6,   # subnormal halves
        np.array([65504, 65519.99, 65520, 65536, 1e9, -1e9, 0.0, -0.0, 2 ** -25, 2 ** -24,
                  3 * 2 ** -25, np.inf, -np.inf], np.float32),
        # exact ties between two halves
        (np.arange(1, 2000, dtype=np.float32) + 0.5) * 2 ** -10,
    ])
    got, bits = oracle.round_f16(x)
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16)
    assert np.array_equal(bits, ref.view(np.uint16))
    assert np.array_equal(got, ref.astype(np.float32))


def test_round_bf16_matches_torch(oracle):
    rng = np.random.default_rng(1)
    x = np.concatenate([
        rng.standard_normal(200000).astype(np.float32) * 100,
        np.array([0.0, -0.0, 1e38, 3.4e38, -3.4e38, 1e-40, np.inf, -np.inf], np.float32),
        (np.arange(1, 3000, dtype=np.float32) * 2 ** -7 + 2 ** -8 * 0.5) * 4,
    ])
    got, bits = oracle.round_bf16(x)
    ref = torch.from_numpy(x).to(torch.bfloat16)
    assert np.array_equal(bits, ref.view(torch.int16).numpy().view(np.uint16))
    assert np.array_equal(got, ref.float().numpy())


# ---------------------------------------------------------------------------
# Pin of the reference-kernel emulator's rounding.  With V rows one-hot
# (V[j] = e_j) and integer Q, K (exact fp32 scores), the emulator's output
# exposes every rounded P: O[i][j] = round_out(P_j * alpha-rescaled / l).  The
# restatement below follows the reference's arithmetic in numpy
# (online_softmax.cuh:13-19 p = exp2(s*c - m*c), :17-19 alpha, :89-152 the
# rescale and the sum l of the unrounded p; forward_v6_mma.cuh:19-38 P
# rounded RNE to the input type before P V; :206-234 O normalised in fp32 and
# rounded), tile by tile.  The emulator must equal it on every element, and a
# restatement that rounds P to the other 16-bit type must not.


def _round_t(x, dt):
    t = torch.from_numpy(np.ascontiguousarray(x, np.float32))
    return t.to(dt).float().numpy()


def _restated_one_hot(qi, ki, scale, p_dtype, o_dtype, block_n=64, l_rounded=False):
    """Emulator arithmetic for V = one-hot rows, restated per tile in numpy
    (l_rounded: a planted mistake, l summed over the rounded P)."""
    N, D = ki.shape
    s = (qi.astype(np.int64) @ ki.astype(np.int64).T).astype(np.float64)  # exact
    c = np.float32(np.float32(scale) * np.float32(1.4426950408889634))
    out = np.zeros((qi.shape[0], D), np.float32)
    for i in range(qi.shape[0]):
        m = np.float32(-np.inf)
        l = np.float32(0.0)
        acc = np.zeros(D, np.float32)
        for t0 in range(0, N, block_n):
            st = s[i, t0:t0 + block_n]
            mt = np.float32(max(float(m), float(st.max())))
            with np.errstate(invalid="ignore"):
                a_arg = np.float32((m - mt) * c)
            alpha = np.float32(np.exp2(np.float64(a_arg)))
            l = np.float32(l * alpha)
            acc = (acc * alpha).astype(np.float32)
            mc = np.float64(np.float32(mt * c))
            x = (st * np.float64(c) - mc).astype(np.float32)  # fmaf(s, c, -(m*c))
            p = np.exp2(x.astype(np.float64)).astype(np.float32)
            pr = _round_t(p, p_dtype)
            for pj in (pr if l_rounded else p):
                l = np.float32(l + pj)
            acc[t0:t0 + len(st)] = (acc[t0:t0 + len(st)] + pr).astype(np.float32)
            m = mt
        inv = np.float32(np.float32(1.0) / l)
        out[i] = _round_t(acc * inv, o_dtype)
    return out


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("N,D", [(48, 64), (128, 128)])
def test_kernel_numerics_rounding_pinned(oracle, dtype, N, D):
    rng = np.random.default_rng(N + D)
    qi = rng.integers(-3, 4, size=(N, D))
    ki = rng.integers(-3, 4, size=(N, D))
    v = np.zeros((N, D), np.float32)
    v[np.arange(N), np.arange(N)] = 1.0
    scale = 0.05
    tdt, other = ((torch.float16, torch.bfloat16) if dtype == "fp16"
                  else (torch.bfloat16, torch.float16))
    q4 = qi.astype(np.float32)[None, None]
    k4 = ki.astype(np.float32)[None, None]
    eo, _ = oracle.kernel_numerics(q4, k4, v[None, None], scale, False,
                                   oracle.BF16 if dtype == "bf16" else oracle.F16)
    eo = eo[0, 0]
    # every output value is representable in the output type (O is rounded)
    assert np.array_equal(_round_t(eo, tdt), eo)
    ref = _restated_one_hot(qi, ki, scale, tdt, tdt)
    assert np.array_equal(eo, ref)
    # P rounded to the other 16-bit type: visibly different
    wrong = _restated_one_hot(qi, ki, scale, other, tdt)
    assert (wrong[:, :N] != eo[:, :N]).mean() > 0.1
    # l summed over the rounded P instead of the unrounded p: also visible
    wrong_l = _restated_one_hot(qi, ki, scale, tdt, tdt, l_rounded=True)
    assert (wrong_l[:, :N] != eo[:, :N]).mean() > 0.01
