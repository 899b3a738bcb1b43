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
from helpers import LSE_TOL, MAX_ABS_TOL, case_seed, err_stats, make_qkv, to_np32
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


# ---- seeded hard inputs and plan boundaries ----
#
# Generators of the kinds of problem that found faults the fixed cases had
# missed: outlier keys far above the rest, attention sinks over long rows,
# huge |V|, all-zero Q, identical keys, per-tensor BNHD / padded layouts and
# outputs written into strided views of a larger buffer; and N placed where
# the work plan switches (8-wave thresholds, bf16's tile limit, pair-mode
# bounds, exactly two q-tiles per CU).  The bar against the emulated
# reference kernel allows half an output ulp of the row on top of 2x its
# max-abs error: on ~100 sampled rows the maximum is often one rounding of
# the output itself.

TD = {"fp16": torch.float16, "bf16": torch.bfloat16}


def _hard_case(case):
    rng = np.random.default_rng(case_seed(3000 + case))
    D = int(rng.choice([64, 128]))
    dtype = str(rng.choice(["fp16", "bf16"]))
    causal = bool(rng.integers(0, 2))
    mode = ["outlier", "sink", "bigv", "zeroq", "dupk", "wide"][case % 6]
    N = int(rng.choice([127, 128, 1000, 2049, 4096, 8191, 12000]))
    B, H = int(rng.integers(1, 3)), int(rng.integers(1, 5))
    scale = None if rng.random() < 0.5 else float(np.exp(rng.uniform(np.log(0.02), np.log(0.6))))
    lay = [str(rng.choice(["bhnd", "bnhd", "padded"])) for _ in range(3)]
    out = str(rng.choice(["fresh", "bnhd_view", "padded_view"]))
    return rng, B, H, N, D, dtype, causal, mode, scale, lay, out


def _hard_inputs(rng, case, B, H, N, D, dtype, mode):
    g = torch.Generator().manual_seed(case_seed(3100 + case))
    sigma = 6.0 if mode == "wide" else 1.0
    q = torch.randn(B, H, N, D, generator=g) * (0.1 if mode in ("outlier", "sink") else sigma)
    k = torch.randn(B, H, N, D, generator=g) * (0.1 if mode in ("outlier", "sink") else sigma)
    v = torch.randn(B, H, N, D, generator=g)
    vmul = 1.0
    if mode in ("outlier", "sink"):
        q[..., 0] = 8.0
        k[..., 0] = 0.0
        keys = [0] if mode == "sink" else rng.integers(0, N, size=int(rng.integers(1, 6))).tolist()
        for j in keys:
            rise = float(rng.uniform(8, 30) if mode == "sink" else rng.uniform(10, 200))
            k[:, :, j, 0] = rise * math.log(2) * math.sqrt(D) / 8.0
    elif mode == "bigv":
        vmul = 5e3 if dtype == "fp16" else 1e25
    elif mode == "zeroq":
        q.zero_()
    elif mode == "dupk":
        k[:] = k[:, :, :1, :]
    return q.to(TD[dtype]), k.to(TD[dtype]), (v * vmul).to(TD[dtype]), vmul


def _place(t, layout):
    if layout == "bnhd":
        return t.permute(0, 2, 1, 3).contiguous().to(DEV).permute(0, 2, 1, 3)
    if layout == "padded":
        B, H, N, D = t.shape
        buf = torch.zeros(B, H, N, D + 64, dtype=t.dtype)
        buf[..., :D] = t
        return buf.to(DEV)[..., :D]
    return t.to(DEV)


def _check_rows(oracle, q, k, v, o, lse, scale, causal, dtype, vmul, rng):
    B, H, N, D = q.shape
    rows = {0, 1, 63, 64, 65, 127, 128, N - 1, N // 2}
    rows |= set(rng.integers(0, N, size=24).tolist())
    rows = sorted(r for r in rows if 0 <= r < N)
    bhs = sorted({0, B * H - 1, (B * H) // 2})
    sel_bh = np.array([b for b in bhs for _ in rows], np.int32)
    sel_row = np.array([r for _ in bhs for r in rows], np.int32)
    qn, kn, vn = (to_np32(t.reshape(1, B * H, N, D)) for t in (q, k, v))
    ref_o, ref_lse = oracle.attn_rows_f64(qn, kn, vn, scale, causal, sel_bh, sel_row)
    emu_o, _ = oracle.kernel_numerics_rows(qn, kn, vn, scale, causal, sel_bh, sel_row,
                                           oracle.BF16 if dtype == "bf16" else oracle.F16)
    got = to_np32(o.reshape(B * H, N, D))[sel_bh, sel_row] / vmul
    ref_o, emu_o = ref_o / vmul, emu_o / vmul
    got_lse = to_np32(lse.reshape(B * H, N))[sel_bh, sel_row].astype(np.float64)
    mx, mean = err_stats(got, ref_o)
    emx, emean = err_stats(emu_o, ref_o)
    lse_err = float(np.abs(got_lse - ref_lse).max())
    top = float(np.abs(ref_o).max())
    half_ulp = top * (2.0 ** -11 if dtype == "fp16" else 2.0 ** -8)
    _note(f"  {len(sel_row)} rows: max_abs={mx:.3e} mean_abs={mean:.3e} "
          f"(ref-kernel emu {emx:.3e}/{emean:.3e}) lse={lse_err:.3e}")
    assert mx <= MAX_ABS_TOL * max(1.0, top)
    assert mx <= 2 * emx + half_ulp + 1e-6 and mean <= 2 * emean + 1e-6
    assert lse_err <= LSE_TOL


@pytest.mark.parametrize("case", range(36))
def test_random_hard_inputs_vs_oracle(fa, oracle, case):
    rng, B, H, N, D, dtype, causal, mode, scale, lay, out = _hard_case(case)
    _note(f"case hard#{case}: {B}x{H}x{N}x{D} {dtype} causal={causal} mode={mode} "
          f"scale={scale} layout={lay} out={out}")
    q, k, v, vmul = _hard_inputs(rng, case, B, H, N, D, dtype, mode)
    qd, kd, vd = _place(q, lay[0]), _place(k, lay[1]), _place(v, lay[2])
    o_arg, buf = None, None
    if out == "bnhd_view":
        buf = torch.full((B, N, H, D), 7.0, dtype=TD[dtype], device=DEV)
        o_arg = buf.permute(0, 2, 1, 3)
    elif out == "padded_view":
        buf = torch.full((B, H, N, D + 32), 7.0, dtype=TD[dtype], device=DEV)
        o_arg = buf[..., :D]
    o, lse = fa.forward(qd, kd, vd, o_arg, causal=causal, softmax_scale=scale, return_lse=True)
    o2 = fa.forward(qd, kd, vd, causal=causal, softmax_scale=scale)
    o1, lse1 = fa.forward(qd, kd, vd, causal=causal, softmax_scale=scale, return_lse=True,
                          split_kv=False)
    torch.cuda.synchronize()
    if o_arg is not None:
        assert o.data_ptr() == o_arg.data_ptr()
        if out == "padded_view":
            assert bool((buf[..., D:] == 7.0).all().item())
    assert torch.isfinite(o).all().item() and torch.isfinite(lse).all().item()
    assert torch.equal(o, o2)
    _vs_unsplit(o / vmul, lse, o1 / vmul, lse1, dtype)
    sc = scale if scale is not None else 1.0 / math.sqrt(D)
    _check_rows(oracle, q, k, v, o, lse, sc, causal, dtype, vmul, rng)


def _boundary_case(case):
    rng = np.random.default_rng(case_seed(3200 + case))
    D = int(rng.choice([64, 128]))
    dtype = str(rng.choice(["fp16", "bf16"]))
    causal = bool(rng.random() < 0.75)
    B = int(rng.choice([1, 2, 4]))
    H = int(rng.choice([1, 2, 3, 4, 6, 8, 12, 16, 24, 32]))
    bh = B * H
    kind = case % 4
    if kind == 0:    # 8-wave thresholds
        N = int(rng.choice([2047, 2048, 2049, 8191, 8192, 8193]))
    elif kind == 1:  # bf16's tile limit: B*H*ceil(N/128) around 192
        N = max(1, (int(rng.choice([191, 192, 193])) // bh) * 128 - int(rng.integers(0, 127)))
    elif kind == 2:  # pair-mode bounds: 128-row q-tiles around 0.75 and 2 per CU
        t = int(rng.choice([191, 192, 193, 511, 512, 513]))
        N = max(1, int(math.ceil(t / bh)) * 128 - int(rng.integers(0, 127)))
    else:            # exactly two q-tiles per CU (the XCD placement table when B*H % 8 == 0)
        N = max(1, (512 // bh) * 128 - int(rng.integers(0, 127)))
    N = max(1, min(N, 24 * 2 ** 20 // D // bh))
    sigma = float(rng.choice([1.0, 3.0]))
    return rng, B, H, N, D, dtype, causal, sigma


@pytest.mark.parametrize("case", range(36))
def test_random_plan_boundaries_vs_oracle(fa, oracle, lib, case):
    import ctypes

    rng, B, H, N, D, dtype, causal, sigma = _boundary_case(case)
    q, k, v = make_qkv(B, H, N, D, dtype, seed=case_seed(3300 + case), qk_sigma=sigma, device=DEV)
    p = A.params_from_tensors(q, k, v, torch.empty_like(q), None, causal)
    pl = A.FaFwdPlan()
    assert lib.fa_fwd_plan(ctypes.byref(p), int(fa.device_info(0)["compute_units"]),
                           ctypes.byref(pl)) == A.FA_OK
    kind = ("pair" if pl.key_halves == 2 else "table" if pl.xcd_heads
            else "split" if pl.n_items else "plain")
    _note(f"case boundary#{case}: {B}x{H}x{N}x{D} {dtype} causal={causal} sigma={sigma} "
          f"plan={kind} BM={pl.block_rows}")
    o, lse = fa.forward(q, k, v, causal=causal, return_lse=True)
    o1, lse1 = fa.forward(q, k, v, causal=causal, return_lse=True, split_kv=False)
    torch.cuda.synchronize()
    assert torch.isfinite(o).all().item() and torch.isfinite(lse).all().item()
    if kind == "split":
        _vs_unsplit(o, lse, o1, lse1, dtype)
    else:
        assert torch.equal(o, o1) and torch.equal(lse, lse1)
    _check_rows(oracle, q, k, v, o, lse, 1.0 / math.sqrt(D), causal, dtype, 1.0, rng)
