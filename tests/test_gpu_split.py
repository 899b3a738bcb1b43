"""GPU parity of split-KV (fa_fwd_ws): long key ranges of a q-tile computed
by several workgroups whose fp32 partials are merged by a second kernel.

Every case first asks the library (fa_fwd_plan with this device's CU count)
for its plan and asserts that it really splits, so these tests cannot pass
on the unsplit path by accident.  The split result is checked against the
fp64 oracle and the reference-kernel emulator (same bars as the unsplit
kernel), against the unsplit result of the same inputs, and for the merge's
own edge cases: chunks whose rows see no key, score jumps between chunks,
ragged tails, strided outputs inside a larger buffer, LSE, graph capture.
Direct C-ABI calls (ctypes, raw device pointers) cover the workspace
contract: size query, rejection of a short or misaligned workspace with the
output untouched, and the timed variant.
"""
from __future__ import annotations

import ctypes
import math

import numpy as np
import pytest
import torch

import abi_ctypes as A
from helpers import LSE_TOL, MAX_ABS_TOL, case_seed, err_stats, make_config, make_qkv, to_np32
from test_gpu_parity import _check_against_oracle, _sample_rows, _scale_keys

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _note(msg):
    print(msg, flush=True)


@pytest.fixture(scope="module")
def lib():
    return A.load()


@pytest.fixture(scope="module")
def cus(fa):
    return int(fa.device_info(0)["compute_units"])


def _plan(lib, cus, q, k, v, o, causal):
    p = A.params_from_tensors(q, k, v, o, None, causal)
    pl = A.FaFwdPlan()
    assert lib.fa_fwd_plan(ctypes.byref(p), cus, ctypes.byref(pl)) == A.FA_OK
    return pl


def _assert_split(lib, cus, q, k, v, causal):
    pl = _plan(lib, cus, q, k, v, torch.empty_like(q), causal)
    _note(f"  plan: BM={pl.block_rows} items={pl.n_items} slots={pl.n_slots} "
          f"merge={pl.n_merge} workspace={pl.workspace_bytes}")
    assert pl.n_items > 0 and pl.n_merge > 0, "expected a split plan on this device"
    return pl


def _both(fa, q, k, v, causal, scale=None):
    o, lse = fa.forward(q, k, v, causal=causal, softmax_scale=scale, return_lse=True)
    o1, lse1 = fa.forward(q, k, v, causal=causal, softmax_scale=scale, return_lse=True,
                          split_kv=False)
    torch.cuda.synchronize()
    return o, lse, o1, lse1


def _vs_unsplit(o, lse, o1, lse1, dtype):
    """Split and unsplit differ where the exponent offsets sit (each chunk
    has its own), so P rounds differently before P.V (2^-11 relative for
    fp16, 2^-8 for bf16, per term), and by the fp32 merge.  A merge mistake
    (a wrong weight, slot or row) shows as an error of the order of |O|.
    LSE: fp16 sums the rounded P (relative error <= 2^-11 per term, so each
    of ln l_split and ln l_unsplit is within 2^-11 of the exact value); bf16
    sums the unrounded fp32 p on both paths."""
    d = (o.float() - o1.float()).abs()
    u = 2.0 ** -9 if dtype == "fp16" else 2.0 ** -6
    n_bad = int((d > u * (1.0 + o1.float().abs())).sum().item())
    dl = (lse - lse1).abs().max().item()
    _note(f"  vs unsplit: max|dO|={d.max().item():.3e} mean|dO|={d.mean().item():.3e} "
          f"over-bound={n_bad} max|dLSE|={dl:.3e}")
    assert n_bad == 0
    assert d.mean().item() <= u / 8
    assert dl <= (2.0 ** -10 + 1e-5 if dtype == "fp16" else 1e-4)


@pytest.mark.parametrize("causal", [False, True], ids=["noncausal", "causal"])
@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("N", [700, 1024, 1537])
def test_split_small_vs_oracle(fa, oracle, lib, cus, N, D, dtype, causal):
    """One or two heads: the unsplit grid would occupy a few CUs, so every
    q-tile beyond 8 key tiles is split.  Ragged N included."""
    H = 2 if N < 1500 else 1
    _note(f"case split small N={N} D={D} {dtype} causal={causal}")
    q, k, v = make_qkv(1, H, N, D, dtype, seed=case_seed(900 + N + D), device=DEV)
    _assert_split(lib, cus, q, k, v, causal)
    o, lse, o1, lse1 = _both(fa, q, k, v, causal)
    _check_against_oracle(oracle, q, k, v, o, lse, causal, 1.0 / math.sqrt(D), dtype)
    _vs_unsplit(o, lse, o1, lse1, dtype)


@pytest.mark.parametrize("pattern", ["jump", "ramp", "half", "drop"])
@pytest.mark.parametrize("causal", [False, True], ids=["noncausal", "causal"])
@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
def test_split_score_jumps_vs_oracle(fa, oracle, lib, cus, pattern, causal, dtype):
    """Scores that jump between key tiles put the chunks' offsets m_c far
    apart ("drop": the first chunk holds the max, later chunks' weights
    underflow toward 0; "ramp": the last chunk dominates)."""
    _note(f"case split jumps pattern={pattern} {dtype} causal={causal}")
    N, D = 1280, 128
    q, k, v = make_qkv(1, 1, N, D, dtype, seed=case_seed(901), device="cpu")
    tdt = torch.float16 if dtype == "fp16" else torch.bfloat16
    k = _scale_keys(k, pattern).to(tdt)
    q, k, v = q.to(DEV), k.to(DEV), v.to(DEV)
    _assert_split(lib, cus, q, k, v, causal)
    o, lse, o1, lse1 = _both(fa, q, k, v, causal)
    _check_against_oracle(oracle, q, k, v, o, lse, causal, 1.0 / math.sqrt(D), dtype,
                          contract=False)


@pytest.mark.parametrize("scale", [0.01, 3.0])
def test_split_softmax_scale_vs_oracle(fa, oracle, lib, cus, scale):
    """Flat (scale 0.01) and peaked (scale 3) rows through the merge."""
    _note(f"case split scale={scale}")
    N, D = 1024, 64
    q, k, v = make_qkv(1, 2, N, D, "fp16", seed=case_seed(902), device=DEV)
    _assert_split(lib, cus, q, k, v, True)
    o, lse, o1, lse1 = _both(fa, q, k, v, True, scale)
    _check_against_oracle(oracle, q, k, v, o, lse, True, scale, "fp16", contract=False)


def test_split_c5r_quarter_heads_vs_oracle_and_unsplit(fa, oracle, lib, cus):
    """C5r's shape and inputs (N3000 causal fp16, Q, K ~ N(0, 3^2)) with 4 of
    its 16 heads, which the plan splits into up to 3 chunks per q-tile:
    sampled rows against the oracle and the reference-kernel emulator, and
    split == unsplit within two roundings."""
    _note("case split C5r/4")
    B, H, N, D = 1, 4, 3000, 128
    q, k, v = make_qkv(B, H, N, D, "fp16", seed=case_seed(5), qk_sigma=3.0, device=DEV)
    pl = _assert_split(lib, cus, q, k, v, True)
    assert pl.block_rows == 128
    o, lse, o1, lse1 = _both(fa, q, k, v, True)
    assert torch.isfinite(o).all().item()
    _vs_unsplit(o, lse, o1, lse1, "fp16")
    rng = np.random.default_rng(5)
    heads, sel_bh, sel_row = _sample_rows(N, H, rng, n_random=48)
    qn, kn, vn = to_np32(q), to_np32(k), to_np32(v)
    scale = 1.0 / math.sqrt(D)
    ref_o, ref_lse = oracle.attn_rows_f64(qn, kn, vn, scale, True, sel_bh, sel_row)
    emu_o, _ = oracle.kernel_numerics_rows(qn, kn, vn, scale, True, sel_bh, sel_row, oracle.F16)
    got_o = to_np32(o.reshape(H, N, D))[sel_bh, sel_row]
    got_lse = to_np32(lse.reshape(H, N))[sel_bh, sel_row]
    mx, mean = err_stats(got_o, ref_o)
    emx, emean = err_stats(emu_o, ref_o)
    lse_err = float(np.abs(got_lse.astype(np.float64) - ref_lse).max())
    _note(f"  sampled {len(sel_row)} rows: max_abs={mx:.3e} mean_abs={mean:.3e} "
          f"(ref-kernel emu {emx:.3e}/{emean:.3e}) lse={lse_err:.3e}")
    assert mx <= MAX_ABS_TOL
    assert mx <= 2 * emx + 1e-6 and mean <= 2 * emean + 1e-6
    assert lse_err <= LSE_TOL


@pytest.mark.parametrize("B,H,N,D,dtype,causal,kind", [
    (1, 2, 128, 64, "fp16", True, "plain"),     # 16x16x32 4-wave, checked pass, kept p
    (1, 2, 128, 64, "fp16", False, "plain"),    # 32x32x16 4-wave D = 64, redone pass
    (1, 2, 128, 64, "bf16", True, "plain"),     # bf16's optimistic pass redone
    (1, 2, 128, 64, "bf16", False, "plain"),
    (1, 2, 2048, 128, "fp16", False, "plain"),  # 8-wave, redone pass, kept p
    (1, 8, 3000, 128, "fp16", True, "pair"),
    (1, 8, 3000, 128, "bf16", True, "pair"),
    (1, 1, 4096, 128, "fp16", False, "split"),
])
def test_offset_move_of_128_log2_units(fa, oracle, lib, cus, B, H, N, D, dtype, causal, kind):
    """Every row's max rises ~128 log2 units on one key tile (a single key).
    The checked pass moves the offset by that much; where it keeps the tile's
    fp32 p and rescales them by alpha = 2^-128 instead of computing them
    again, alpha is below the normal range and exp2 returns 0 for it, which
    zeroes the tile that holds the row's max (O = 0, LSE = -inf).  Moves of
    126 log2 units or more must recompute p.  The jump key sits in key tile 1
    (N = 128) or 2 (the pair-mode halves take alternate tiles, so tile 2 is
    the second tile of a half)."""
    _note(f"case offset move 128: {B}x{H}x{N}x{D} {dtype} causal={causal} ({kind})")
    tdt = torch.float16 if dtype == "fp16" else torch.bfloat16
    gen = torch.Generator().manual_seed(case_seed(791))
    q = torch.randn(B, H, N, D, generator=gen) * 0.1
    k = torch.randn(B, H, N, D, generator=gen) * 0.1
    v = torch.randn(B, H, N, D, generator=gen)
    jk = 64 if N == 128 else 128
    scale = 1.0 / math.sqrt(D)
    q[..., 0] = 32.0
    k[..., 0] = 0.0
    k[:, :, jk, 0] = 128.0 / (32.0 * scale * math.log2(math.e))
    q, k, v = (t.to(tdt) for t in (q, k, v))
    rise = 32.0 * float(k[0, 0, jk, 0]) * scale * math.log2(math.e)
    assert 126.5 < rise < 129.5, rise
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    if kind != "plain":
        pl = _plan(lib, cus, qd, kd, vd, torch.empty_like(qd), causal)
        assert ("pair" if pl.key_halves == 2 else "split" if pl.n_items else "other") == kind
    o, lse = fa.forward(qd, kd, vd, causal=causal, return_lse=True, split_kv=kind != "plain")
    torch.cuda.synchronize()
    assert torch.isfinite(o).all().item() and torch.isfinite(lse).all().item()
    rng = np.random.default_rng(791)
    _, sel_bh, sel_row = _sample_rows(N, B * H, rng, n_random=32)
    qn, kn, vn = (to_np32(t.reshape(1, B * H, N, D)) for t in (q, k, v))
    ref_o, ref_lse = oracle.attn_rows_f64(qn, kn, vn, scale, causal, sel_bh, sel_row)
    got = to_np32(o.reshape(B * H, N, D))[sel_bh, sel_row].astype(np.float64)
    got_lse = to_np32(lse.reshape(B * H, N))[sel_bh, sel_row].astype(np.float64)
    row_scale = np.maximum(1.0, np.abs(ref_o).max(axis=-1, keepdims=True))
    rel = float((np.abs(got - ref_o) / row_scale).max())
    lse_err = float(np.abs(got_lse - ref_lse).max())
    _note(f"  {len(sel_row)} rows: max rel-to-row err={rel:.3e} lse_err={lse_err:.3e}")
    assert rel <= 1e-2, rel
    assert lse_err <= LSE_TOL, lse_err


def _two_key_rows(B, H, N, D, keys, seed):
    """bf16 Q, K, V whose every row scores ~0 except at `keys` {index: log2
    units above the rest}."""
    gen = torch.Generator().manual_seed(case_seed(seed))
    q = torch.randn(B, H, N, D, generator=gen) * 0.1
    k = torch.randn(B, H, N, D, generator=gen) * 0.1
    v = torch.randn(B, H, N, D, generator=gen)
    scale = 1.0 / math.sqrt(D)
    q[..., 0] = 8.0
    k[..., 0] = 0.0
    for j, rise in keys.items():
        k[:, :, j, 0] = rise * math.log(2) / (8.0 * scale)
    return tuple(t.to(torch.bfloat16) for t in (q, k, v)), scale


@pytest.mark.parametrize("kind", ["split", "pair"])
def test_partials_far_below_the_row_max(fa, oracle, lib, cus, kind):
    """bf16's optimistic pass keeps the offset of a partial's first tile, so
    a partial (a split chunk, a pair half) can hold a row sum of ~2^118 at an
    offset ~126 log2 units below another partial's.  Key A (118 units above
    the rest) lies inside one partial after its first tile, key B (126.5
    units) opens the next one: A holds 2^-8.5 of the row.  Weighting the
    unnormalised partial by exp2(offset difference) = 2^-126.5 underflowed
    to 0 and lost A (LSE 2.75e-3 low); partials are normalised by their own
    sums before they are combined."""
    if kind == "split":
        B, H, N, D, causal = 1, 1, 4096, 128, False
    else:
        B, H, N, D, causal = 1, 8, 3000, 128, True
    (q, k, v), scale = _two_key_rows(B, H, N, D, {}, 795)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    pl = _plan(lib, cus, qd, kd, vd, torch.empty_like(qd), causal)
    if kind == "split":
        assert pl.n_items > 0 and pl.n_merge > 0
        ends = sorted({pl.tile_end[i] for i in range(pl.n_items)
                       if pl.q_tile[i] == 0 and pl.tile_begin[i] == 0})
        assert ends and ends[0] < (N + 63) // 64, "expected q-tile 0 in several chunks"
        a_key, b_key = 100, 64 * ends[0] + 5  # A in chunk 0 after its first tile; B opens chunk 1
    else:
        assert pl.key_halves == 2
        a_key, b_key = 130, 70  # A in tile 2 (the even half's second), B in tile 1 (the odd half's first)
    _note(f"case partials far below the max ({kind}): {B}x{H}x{N}x{D} keys A={a_key} B={b_key}")
    (q, k, v), scale = _two_key_rows(B, H, N, D, {a_key: 118.0, b_key: 126.5}, 795)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    o, lse = fa.forward(qd, kd, vd, causal=causal, return_lse=True)
    torch.cuda.synchronize()
    assert torch.isfinite(o).all().item() and torch.isfinite(lse).all().item()
    rng = np.random.default_rng(795)
    _, sel_bh, sel_row = _sample_rows(N, B * H, rng, n_random=32)
    qn, kn, vn = (to_np32(t.reshape(1, B * H, N, D)) for t in (q, k, v))
    ref_o, ref_lse = oracle.attn_rows_f64(qn, kn, vn, scale, causal, sel_bh, sel_row)
    got = to_np32(o.reshape(B * H, N, D))[sel_bh, sel_row].astype(np.float64)
    got_lse = to_np32(lse.reshape(B * H, N))[sel_bh, sel_row].astype(np.float64)
    row_scale = np.maximum(1.0, np.abs(ref_o).max(axis=-1, keepdims=True))
    rel = float((np.abs(got - ref_o) / row_scale).max())
    lse_err = float(np.abs(got_lse - ref_lse).max())
    _note(f"  {len(sel_row)} rows: max rel-to-row err={rel:.3e} lse_err={lse_err:.3e}")
    assert rel <= 1e-2, rel
    assert lse_err <= LSE_TOL, lse_err


@pytest.mark.parametrize("causal,N,H,dtype,sigma", [
    (True, 8192, 2, "fp16", 1.0), (False, 4096, 1, "fp16", 1.0),
    (True, 8192, 2, "bf16", 3.0),   # bf16's optimistic pass on wide scores
    (False, 4096, 1, "bf16", 3.0),
], ids=["causal8192", "noncausal4096", "causal8192-bf16-s3", "noncausal4096-bf16-s3"])
def test_split_wide_workgroup_sampled_rows(fa, oracle, lib, cus, causal, N, H, dtype, sigma):
    """8-wave workgroups (BM = 256) with the optimistic pass, split: sampled
    rows against the oracle and the reference-kernel emulator.  bf16 runs
    that pass with no spread test, so Q, K ~ N(0, 3^2) keeps the first
    tile's offset through the rising maxima of a long row."""
    _note(f"case split wide causal={causal} N={N} H={H} {dtype} sigma={sigma}")
    D = 128
    q, k, v = make_qkv(1, H, N, D, dtype, seed=case_seed(903), qk_sigma=sigma, device=DEV)
    pl = _assert_split(lib, cus, q, k, v, causal)
    assert pl.block_rows == 256
    o, lse, o1, lse1 = _both(fa, q, k, v, causal)
    _vs_unsplit(o, lse, o1, lse1, dtype)
    rng = np.random.default_rng(903)
    heads, sel_bh, sel_row = _sample_rows(N, H, rng, n_random=32)
    qn, kn, vn = to_np32(q), to_np32(k), to_np32(v)
    scale = 1.0 / math.sqrt(D)
    ref_o, ref_lse = oracle.attn_rows_f64(qn, kn, vn, scale, causal, sel_bh, sel_row)
    emu_o, _ = oracle.kernel_numerics_rows(qn, kn, vn, scale, causal, sel_bh, sel_row,
                                           oracle.BF16 if dtype == "bf16" else oracle.F16)
    got_o = to_np32(o.reshape(H, N, D))[sel_bh, sel_row]
    got_lse = to_np32(lse.reshape(H, N))[sel_bh, sel_row]
    mx, mean = err_stats(got_o, ref_o)
    emx, emean = err_stats(emu_o, ref_o)
    lse_err = float(np.abs(got_lse.astype(np.float64) - ref_lse).max())
    _note(f"  sampled {len(sel_row)} rows: max_abs={mx:.3e} mean_abs={mean:.3e} "
          f"(ref-kernel emu {emx:.3e}/{emean:.3e}) lse={lse_err:.3e}")
    # bf16 with wide scores: peaked rows put |O| above 1 (the bar scales)
    o_scale = max(1.0, float(np.abs(ref_o).max())) if dtype == "bf16" else 1.0
    assert mx <= MAX_ABS_TOL * o_scale
    assert mx <= 2 * emx + 1e-6 and mean <= 2 * emean + 1e-6
    assert lse_err <= LSE_TOL


@pytest.mark.parametrize("B,H,N,dtype", [(1, 4, 8192, "fp16"), (1, 2, 8192, "bf16")],
                         ids=["S2-fp16", "S4-bf16"])
def test_split_full_tensor_through_fa_fwd_ws(fa, oracle, lib, cus, B, H, N, dtype):
    """The bench's few-head causal shapes S2 and S4 (N = 8192, BASELINE-sized
    rows), called through the C ABI's fa_fwd_ws with a workspace of exactly
    fa_fwd_workspace_size bytes: the plan must split (chunks and the merge
    kernel run), and every element of O and the LSE is checked against the
    fp64 oracle and the reference-kernel emulator at the contract bars
    (benchmark/cpp/correctness_v6.cu:74-104 is the reference's gate)."""
    _note(f"case split full tensor {B}x{H}x{N}x128 {dtype} causal via fa_fwd_ws")
    D = 128
    q, k, v = make_qkv(B, H, N, D, dtype, seed=case_seed(907 + H), device=DEV)
    pl = _assert_split(lib, cus, q, k, v, True)
    o = torch.full_like(q, float("nan"))
    lse = torch.full((B, H, N), float("nan"), dtype=torch.float32, device=DEV)
    p = A.params_from_tensors(q, k, v, o, lse, True)
    need = ctypes.c_uint64(0)
    assert lib.fa_fwd_workspace_size(ctypes.byref(p), ctypes.byref(need)) == A.FA_OK
    assert need.value == pl.workspace_bytes > 0
    ws = torch.empty(need.value, dtype=torch.uint8, device=DEV)
    assert lib.fa_fwd_ws(ctypes.byref(p), ctypes.c_void_p(ws.data_ptr()), need.value,
                         _stream()) == A.FA_OK, lib.fa_last_error()
    torch.cuda.synchronize()
    _check_against_oracle(oracle, q, k, v, o, lse, True, 1.0 / math.sqrt(D), dtype)
    o1, lse1 = fa.forward(q, k, v, causal=True, return_lse=True, split_kv=False)
    torch.cuda.synchronize()
    _vs_unsplit(o, lse, o1, lse1, dtype)


def test_split_strided_output_in_padded_buffer(fa, oracle, lib, cus):
    """BNHD views with a padded seq stride for Q, K, V and O; O lives inside a
    NaN-filled buffer: the split kernel and the merge write exactly the view."""
    _note("case split strided")
    B, H, N, D = 1, 2, 1000, 64
    q, k, v = make_qkv(B, H, N, D, "bf16", seed=case_seed(904), device=DEV)

    def bnhd(t, pad):
        buf = torch.full((B, N, H, D + pad), float("nan"), dtype=t.dtype, device=DEV)
        view = buf[..., :D].permute(0, 2, 1, 3)
        view.copy_(t)
        return buf, view

    _, qv = bnhd(q, 8)
    _, kv = bnhd(k, 16)
    _, vv = bnhd(v, 0)
    obuf, ov = bnhd(torch.zeros_like(q), 24)
    obuf.fill_(float("nan"))
    _assert_split(lib, cus, qv, kv, vv, True)
    out, lse = fa.forward(qv, kv, vv, ov, causal=True, return_lse=True)
    torch.cuda.synchronize()
    assert out.data_ptr() == ov.data_ptr()
    assert torch.isnan(obuf[..., D:]).all().item(), "padding of O was written"
    _check_against_oracle(oracle, q, k, v, ov, lse, True, 1.0 / math.sqrt(D), "bf16")


def test_split_deterministic_and_graph_replay(fa, lib, cus):
    """Split results are deterministic (no atomics), and a captured graph
    (workspace from the graph's pool) replays to the eager result, several
    times, with eager work in between."""
    _note("case split graph")
    q, k, v = make_qkv(1, 4, 2000, 128, "fp16", seed=case_seed(905), device=DEV)
    _assert_split(lib, cus, q, k, v, True)
    ref = fa.forward(q, k, v, causal=True)
    again = fa.forward(q, k, v, causal=True)
    torch.cuda.synchronize()
    assert torch.equal(ref, again)
    o = torch.empty_like(q)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fa.forward(q, k, v, o, causal=True)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        fa.forward(q, k, v, o, causal=True)
    for rep in range(3):
        o.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(o, ref), f"replay {rep}"
        e = fa.forward(q, k, v, causal=True, split_kv=False)
        torch.cuda.synchronize()
        assert torch.isfinite(e).all().item()


# ------------------------------------------------------------ the C ABI directly


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def test_abi_workspace_contract(fa, lib, cus):
    """fa_fwd_workspace_size, fa_fwd_ws and fa_fwd_ws_timed through ctypes."""
    _note("case split abi")
    q, k, v = make_qkv(1, 2, 1024, 128, "fp16", seed=case_seed(906), device=DEV)
    o = torch.full_like(q, float("nan"))
    lse = torch.empty((1, 2, 1024), dtype=torch.float32, device=DEV)
    p = A.params_from_tensors(q, k, v, o, lse, True)
    need = ctypes.c_uint64(0)
    assert lib.fa_fwd_workspace_size(ctypes.byref(p), ctypes.byref(need)) == A.FA_OK
    pl = _plan(lib, cus, q, k, v, o, True)
    assert need.value == pl.workspace_bytes > 0
    ws = torch.empty(need.value + 256, dtype=torch.uint8, device=DEV)
    torch.cuda.synchronize()

    # rejected before any launch: O keeps its NaN fill
    assert lib.fa_fwd_ws(ctypes.byref(p), None, 0, _stream()) == A.FA_ERR_NULL
    assert lib.fa_fwd_ws(ctypes.byref(p), ctypes.c_void_p(ws.data_ptr()), need.value - 1,
                         _stream()) == A.FA_ERR_ARG
    assert "smaller than" in lib.fa_last_error().decode()
    assert lib.fa_fwd_ws(ctypes.byref(p), ctypes.c_void_p(ws.data_ptr() + 8), need.value,
                         _stream()) == A.FA_ERR_STRIDE
    torch.cuda.synchronize()
    assert torch.isnan(o).all().item()

    # exact size, through fa_fwd_ws, equals the torch path (same plan)
    assert lib.fa_fwd_ws(ctypes.byref(p), ctypes.c_void_p(ws.data_ptr()), need.value,
                         _stream()) == A.FA_OK
    torch.cuda.synchronize()
    ref, ref_lse = fa.forward(q, k, v, causal=True, return_lse=True)
    torch.cuda.synchronize()
    assert torch.equal(o, ref) and torch.equal(lse, ref_lse)

    # LSE optional; timed variant
    o.fill_(float("nan"))
    p2 = A.params_from_tensors(q, k, v, o, None, True)
    ms = ctypes.c_float(0.0)
    assert lib.fa_fwd_ws_timed(ctypes.byref(p2), ctypes.c_void_p(ws.data_ptr()), need.value,
                               _stream(), ctypes.byref(ms)) == A.FA_OK
    torch.cuda.synchronize()
    assert ms.value > 0.0
    assert torch.equal(o, ref)

    # the plain entry point ignores the split and still matches the unsplit torch path
    o.fill_(float("nan"))
    assert lib.fa_fwd(ctypes.byref(p2), _stream()) == A.FA_OK
    torch.cuda.synchronize()
    assert torch.equal(o, fa.forward(q, k, v, causal=True, split_kv=False))


def test_abi_unsplit_problem_needs_no_workspace(fa, lib):
    """C3-sized problems need no workspace: fa_fwd_ws(NULL, 0) is fa_fwd."""
    _note("case split abi unsplit")
    name = "C2"
    q, k, v, causal, _ = make_config(name, device=DEV)
    o = torch.empty_like(q)
    p = A.params_from_tensors(q, k, v, o, None, causal)
    need = ctypes.c_uint64(1)
    assert lib.fa_fwd_workspace_size(ctypes.byref(p), ctypes.byref(need)) == A.FA_OK
    assert need.value == 0
    assert lib.fa_fwd_ws(ctypes.byref(p), None, 0, _stream()) == A.FA_OK
    torch.cuda.synchronize()
    assert torch.equal(o, fa.forward(q, k, v, causal=causal))


def _assert_pair(lib, cus, q, k, v):
    pl = _plan(lib, cus, q, k, v, torch.empty_like(q), True)
    _note(f"  plan: key_halves={pl.key_halves} items={pl.n_items} xcd_heads={pl.xcd_heads}")
    assert pl.key_halves == 2 and pl.n_items == 0 and pl.workspace_bytes == 0
    return pl


def test_pair_mode_c5r_order_and_workspace_invariance(fa, lib, cus):
    """C5r runs in pair mode (rows against the oracle: the full-tensor config
    test).  Each q-tile is computed by one workgroup whatever its position in
    the grid, and the workspace is not used: the result with a workspace
    equals the one without, and permuting the heads permutes the output and
    LSE, bit for bit."""
    _note("case pair mode C5r")
    q, k, v, causal, _ = make_config("C5r", device=DEV)
    if cus == 256:
        _assert_pair(lib, cus, q, k, v)
    o, lse = fa.forward(q, k, v, causal=True, return_lse=True)
    o2, lse2 = fa.forward(q, k, v, causal=True, return_lse=True, split_kv=False)
    torch.cuda.synchronize()
    assert torch.isfinite(o).all().item()
    assert torch.equal(o, o2) and torch.equal(lse, lse2)
    perm = torch.tensor([5, 12, 0, 9, 3, 15, 7, 1, 10, 14, 2, 8, 13, 4, 11, 6], device=DEV)
    qp, kp, vp = (t[:, perm].contiguous() for t in (q, k, v))
    op, lp = fa.forward(qp, kp, vp, causal=True, return_lse=True)
    torch.cuda.synchronize()
    assert torch.equal(op, o[:, perm]) and torch.equal(lp, lse[:, perm])


@pytest.mark.parametrize("B,H,N", [(1, 16, 8192), (2, 32, 2048), (4, 32, 1024)],
                         ids=["2-heads-per-xcd", "8-heads-per-xcd", "16-heads-per-xcd"])
def test_causal_head_interleave_bitwise_equals_plain_order(fa, cus, B, H, N):
    """Causal grids of several rounds with B*H divisible by 8 run each XCD's
    heads in groups of 4 (all of them when their count is not a multiple of
    4), longest q-tiles of the group's heads first.  Only the order changes:
    outputs and LSE equal, bit for bit, those of the same heads run in small
    slices whose B*H is not divisible by 8 (plain order), and small enough
    (below 0.75 q-tiles per CU) not to run in pair mode."""
    _note(f"case causal head interleave B{B} H{H} N{N}")
    q, k, v = make_qkv(B, H, N, 128, "bf16", seed=case_seed(960), device=DEV)
    o, lse = fa.forward(q, k, v, causal=True, return_lse=True, split_kv=False)
    torch.cuda.synchronize()
    nq = (N + 127) // 128
    width = max(w for w in range(1, 6) if 4 * B * w * nq < 3 * cus and (B * w) % 8 != 0)
    lo = 0
    while lo < H:
        hi = min(H, lo + width)
        if (B * (hi - lo)) % 8 == 0:
            hi -= 1
        sl = slice(lo, hi)
        ph, lh = fa.forward(q[:, sl], k[:, sl], v[:, sl], causal=True, return_lse=True,
                            split_kv=False)
        torch.cuda.synchronize()
        assert torch.equal(o[:, sl], ph), f"heads {lo}..{hi - 1}"
        assert torch.equal(lse[:, sl], lh)
        lo = hi


def _sampled_rows_vs_oracle(oracle, q, k, v, o, lse, dtype, seed, n_random=24):
    B, H, N, D = q.shape
    rng = np.random.default_rng(seed)
    heads, sel_bh, sel_row = _sample_rows(N, B * H, rng, n_random=n_random)
    qn, kn, vn = (to_np32(t.reshape(1, B * H, N, D)) for t in (q, k, v))
    scale = 1.0 / math.sqrt(D)
    ref_o, ref_lse = oracle.attn_rows_f64(qn, kn, vn, scale, True, sel_bh, sel_row)
    emu_o, _ = oracle.kernel_numerics_rows(qn, kn, vn, scale, True, sel_bh, sel_row,
                                           oracle.BF16 if dtype == "bf16" else oracle.F16)
    got_o = to_np32(o.reshape(B * H, N, D))[sel_bh, sel_row]
    got_lse = to_np32(lse.reshape(B * H, N))[sel_bh, sel_row]
    mx, mean = err_stats(got_o, ref_o)
    emx, emean = err_stats(emu_o, ref_o)
    lse_err = float(np.abs(got_lse.astype(np.float64) - ref_lse).max())
    _note(f"  sampled {len(sel_row)} rows: max_abs={mx:.3e} mean_abs={mean:.3e} "
          f"(ref-kernel emu {emx:.3e}/{emean:.3e}) lse={lse_err:.3e}")
    assert mx <= MAX_ABS_TOL
    assert mx <= 2 * emx + 1e-6 and mean <= 2 * emean + 1e-6
    assert lse_err <= LSE_TOL


@pytest.mark.parametrize("B,H,N,D,dtype,sigma", [
    (1, 16, 2200, 64, "bf16", 1.0),   # 288 q-tiles
    (2, 8, 3001, 128, "fp16", 1.0),   # ragged, two batches
    (1, 24, 1500, 64, "fp16", 3.0),   # H not a multiple of 8, peaked rows
    (2, 16, 1300, 128, "bf16", 1.0),
    (1, 8, 3000, 128, "fp16", 3.0),   # 192 q-tiles: the lower end of the range
    (1, 8, 3000, 128, "bf16", 3.0),   # bf16's optimistic pass on wide scores
])
def test_pair_mode_variants_vs_oracle(fa, oracle, lib, cus, B, H, N, D, dtype, sigma):
    """Pair mode at D = 64 and 128, fp16 and bf16, ragged N, several batches:
    sampled rows against the oracle and the reference-kernel emulator; with
    and without a workspace bit for bit (one kernel); and against the same
    heads computed one batch and head at a time (4-wave workgroups, no pair
    mode) within the split-KV bounds (the halves' offsets differ, so P
    rounds differently, and the halves meet in fp32)."""
    _note(f"case pair mode {B}x{H}x{N}x{D} {dtype} sigma={sigma}")
    q, k, v = make_qkv(B, H, N, D, dtype, seed=case_seed(970 + N), qk_sigma=sigma, device=DEV)
    if cus == 256:
        _assert_pair(lib, cus, q, k, v)
    o, lse, o1, lse1 = _both(fa, q, k, v, True)
    assert torch.equal(o, o1) and torch.equal(lse, lse1)
    for b in range(B):
        for h in (0, H // 2, H - 1):
            sl = (slice(b, b + 1), slice(h, h + 1))
            ph, lh = fa.forward(q[sl], k[sl], v[sl], causal=True, return_lse=True,
                                split_kv=False)
            torch.cuda.synchronize()
            _vs_unsplit(o[sl], lse[sl], ph, lh, dtype)
    _sampled_rows_vs_oracle(oracle, q, k, v, o, lse, dtype, 970)


@pytest.mark.parametrize("B,H,N,D,dtype", [
    (4, 16, 1000, 64, "bf16"),   # 8 heads x 8 q-tiles per XCD
    (2, 32, 1024, 128, "fp16"),
    # one head x 64 q-tiles per XCD: neighbouring table positions hold
    # different q-tiles (the 16-bit slot array once made every odd
    # position read its neighbour's q-tile)
    (1, 8, 8191, 128, "bf16"),
    (2, 4, 8191, 64, "fp16"),
])
def test_xcd_table_vs_oracle_and_plain_order(fa, oracle, lib, cus, B, H, N, D, dtype):
    """Grids of exactly two q-tiles per CU run with the XCD placement table:
    a dispatch order only, so the output and LSE equal, bit for bit, those of
    each head launched alone (plain longest-first order on the same 4-wave
    kernel); sampled rows against the oracle and the reference-kernel
    emulator."""
    _note(f"case XCD table {B}x{H}x{N}x{D} {dtype}")
    q, k, v = make_qkv(B, H, N, D, dtype, seed=case_seed(980 + N), device=DEV)
    pl = _plan(lib, cus, q, k, v, torch.empty_like(q), True)
    _note(f"  plan: xcd_heads={pl.xcd_heads} items={pl.n_items} merge={pl.n_merge}")
    if cus == 256:
        assert pl.xcd_heads == B * H // 8 and pl.n_items == 64 and pl.n_merge == 0
    o, lse, o1, lse1 = _both(fa, q, k, v, True)
    assert torch.equal(o, o1) and torch.equal(lse, lse1)
    for h in range(H):
        sl = slice(h, h + 1)
        one = _plan(lib, cus, q[:, sl], k[:, sl], v[:, sl], torch.empty_like(q[:, sl]), True)
        assert one.block_rows == 128 and one.key_halves == 1 and one.xcd_heads == 0
        ph, lh = fa.forward(q[:, sl], k[:, sl], v[:, sl], causal=True, return_lse=True,
                            split_kv=False)
        torch.cuda.synchronize()
        assert torch.equal(o1[:, sl], ph), f"head {h}"
        assert torch.equal(lse1[:, sl], lh)
    _sampled_rows_vs_oracle(oracle, q, k, v, o, lse, dtype, 980)


def test_abi_fa_fwd_pair_graph_capture(fa, lib, cus):
    """fa_fwd (no workspace) on C5r (pair mode), called through the raw C
    ABI inside a captured HIP graph: every replay equals the eager result,
    with eager launches in between."""
    _note("case C ABI pair mode graph capture")
    q, k, v, causal, _ = make_config("C5r", device=DEV)
    o = torch.empty_like(q)
    p = A.params_from_tensors(q, k, v, o, None, causal)
    ref = fa.forward(q, k, v, causal=True, split_kv=False)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        assert lib.fa_fwd(ctypes.byref(p), _stream()) == A.FA_OK
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    assert torch.equal(o, ref)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        assert lib.fa_fwd(ctypes.byref(p), _stream()) == A.FA_OK
    for rep in range(3):
        o.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(o, ref), f"replay {rep}"
        e = fa.forward(q, k, v, causal=True)
        torch.cuda.synchronize()
        assert torch.isfinite(e).all().item()
