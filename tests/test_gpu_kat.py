"""Known-answer tests of the MFMA operand layouts and the transposing LDS read
the forward kernel relies on (re-derived from the reference's MMA KATs,
tests/unit/ptx/test_mma_fragment.cu and tests/unit/loadstore/test_copy_srm.cu,
for v_mfma_f32_32x32x16 instead of mma.sync m16n8k16)."""
from __future__ import annotations

import ctypes
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def kat():
    path = os.path.join(HERE, "kat", "libfa_kat.so")
    L = ctypes.CDLL(path)
    u16p = ctypes.POINTER(ctypes.c_uint16)
    fp = ctypes.POINTER(ctypes.c_float)
    L.kat_mfma_32x32x16.argtypes = [ctypes.c_int, u16p, u16p, fp, fp]
    L.kat_ds_read_tr16.argtypes = [ctypes.POINTER(ctypes.c_int16)]
    L.kat_pack2.argtypes = [ctypes.c_int, fp, ctypes.POINTER(ctypes.c_uint32), fp]
    L.kat_pair.argtypes = [fp, fp, fp]
    L.kat_dma.argtypes = [ctypes.POINTER(ctypes.c_int32)]
    L.kat_xcd_remap.argtypes = [ctypes.c_int, ctypes.POINTER(ctypes.c_int32)]
    L.kat_row_sum.argtypes = [u16p, fp, ctypes.c_int, fp]
    return L


def _bits(x, bf16, oracle):
    vals, bits = (oracle.round_bf16 if bf16 else oracle.round_f16)(np.asarray(x, np.float32))
    return vals, bits


def _run(kat, bf16, a_bits, b_bits, c):
    a_bits = np.ascontiguousarray(a_bits, np.uint16)
    b_bits = np.ascontiguousarray(b_bits, np.uint16)
    c = np.ascontiguousarray(c, np.float32)
    d = np.zeros((32, 32), np.float32)
    u16p = ctypes.POINTER(ctypes.c_uint16)
    fp = ctypes.POINTER(ctypes.c_float)
    rc = kat.kat_mfma_32x32x16(int(bf16), a_bits.ctypes.data_as(u16p), b_bits.ctypes.data_as(u16p),
                               c.ctypes.data_as(fp), d.ctypes.data_as(fp))
    assert rc == 0, f"HIP error {rc}"
    return d


@pytest.mark.parametrize("bf16", [False, True], ids=["f16", "bf16"])
def test_mfma_constant_kat(kat, oracle, bf16):
    """A = 0.5, B = 0.25, C = 1.5 -> every D = 1.5 + K * 0.125 = 3.5 for K = 16
    (the reference's constant case, test_mma_fragment.cu:184-213, also K = 16)."""
    print(f"case mfma constant bf16={bf16}", flush=True)
    _, a = _bits(np.full((32, 16), 0.5), bf16, oracle)
    _, b = _bits(np.full((16, 32), 0.25), bf16, oracle)
    d = _run(kat, bf16, a, b, np.full((32, 32), 1.5))
    assert np.all(d == 3.5)


@pytest.mark.parametrize("bf16", [False, True], ids=["f16", "bf16"])
def test_mfma_pattern_kat(kat, oracle, bf16):
    """Non-integer patterns of test_mma_fragment.cu:76-121 / :236-267:
    A[m][k] = 0.10(m+1) + 0.01(k+1) + 0.003, B[k][n] = 0.07(k+1) - 0.015(n+1) + 0.004,
    C = 0.123, compared with the fp32 sum of the quantised operands (tol 1e-2)."""
    print(f"case mfma pattern bf16={bf16}", flush=True)
    m = np.arange(32)[:, None]
    k = np.arange(16)[None, :]
    A = 0.10 * (m + 1) + 0.01 * (k + 1) + 0.003
    kk = np.arange(16)[:, None]
    n = np.arange(32)[None, :]
    B = 0.07 * (kk + 1) - 0.015 * (n + 1) + 0.004
    av, a = _bits(A, bf16, oracle)
    bv, b = _bits(B, bf16, oracle)
    d = _run(kat, bf16, a, b, np.full((32, 32), 0.123))
    ref = av.astype(np.float64) @ bv.astype(np.float64) + 0.123
    assert np.abs(d - ref).max() <= 1e-2
    # Exactness of the layout: a transposed operand would be far off.
    assert np.abs(d - ref).max() <= 1e-3 * np.abs(ref).max()


@pytest.mark.parametrize("bf16", [False, True], ids=["f16", "bf16"])
def test_mfma_pv_kat(kat, oracle, bf16):
    """PV-MMA pattern of test_copy_srm.cu:1247-1298: p = 0.02(m+1) - 0.01(k+1) + 0.003,
    v = 0.05(row+1) + 0.01(col+1) - 0.002, C = 0."""
    print(f"case mfma pv bf16={bf16}", flush=True)
    m = np.arange(32)[:, None]
    k = np.arange(16)[None, :]
    P = 0.02 * (m + 1) - 0.01 * (k + 1) + 0.003
    row = np.arange(16)[:, None]
    col = np.arange(32)[None, :]
    V = 0.05 * (row + 1) + 0.01 * (col + 1) - 0.002
    pv, p = _bits(P, bf16, oracle)
    vv, v = _bits(V, bf16, oracle)
    d = _run(kat, bf16, p, v, np.zeros((32, 32)))
    ref = pv.astype(np.float64) @ vv.astype(np.float64)
    assert np.abs(d - ref).max() <= 1e-2


def test_ds_read_tr16_lane_map(kat):
    """ds_read_tr_pair: within each 16-lane group G, lane i receives element
    (i & 3) of the four 16-bit words addressed by lane G + 4e + ((i % 16) >> 2),
    e = 0..3, for each of the two reads (the second at +512 bytes)."""
    print("case ds_read_b64_tr_b16 lane map", flush=True)
    out = np.zeros((64, 8), np.int16)
    rc = kat.kat_ds_read_tr16(out.ctypes.data_as(ctypes.POINTER(ctypes.c_int16)))
    assert rc == 0
    for i in range(64):
        G = 16 * (i // 16)
        for half in range(2):
            for e in range(4):
                j = G + 4 * e + ((i % 16) >> 2)
                assert out[i, 4 * half + e] == 256 * half + 4 * j + (i & 3), (i, half, e)


@pytest.mark.parametrize("bf16", [False, True], ids=["f16", "bf16"])
def test_pack2_rne_and_dot2(kat, oracle, bf16):
    """pack2 rounds to nearest even exactly like the oracle's RNE conversion
    (ties, subnormals, overflow); dot2_acc adds both halves to an fp32
    accumulator."""
    print(f"case pack2/dot2 bf16={bf16}", flush=True)
    rng = np.random.default_rng(3)
    vals = rng.standard_normal(128).astype(np.float32)
    special = np.array([0.5 + 2 ** -12, 1 + 2 ** -11, 1 + 3 * 2 ** -11, 1 + 2 ** -8, 1 + 3 * 2 ** -8,
                        65504.0, 65520.0, 1e-6, -2 ** -25, 3.0e-5, 1 + 2 ** -9, -1 - 3 * 2 ** -9],
                       np.float32)
    vals[:special.size] = special
    out = np.zeros(64, np.uint32)
    dot = np.zeros(64, np.float32)
    fp = ctypes.POINTER(ctypes.c_float)
    rc = kat.kat_pack2(int(bf16), vals.ctypes.data_as(fp),
                       out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)), dot.ctypes.data_as(fp))
    assert rc == 0
    ref_vals, ref_bits = (oracle.round_bf16 if bf16 else oracle.round_f16)(vals)
    got_bits = np.stack([out & 0xFFFF, out >> 16], axis=1).reshape(-1).astype(np.uint16)
    assert np.array_equal(got_bits, ref_bits)
    pairs = ref_vals.reshape(64, 2).astype(np.float64)
    finite = np.isfinite(pairs).all(axis=1)
    assert np.allclose(dot[finite], 0.25 + pairs[finite].sum(axis=1), rtol=1e-6, atol=1e-6)


def test_pair_reductions(kat):
    """pair_max / pair_sum combine lanes l and l^32 (the two halves of one
    query row in the 32x32 accumulator layout)."""
    print("case pair reductions", flush=True)
    x = np.random.default_rng(4).standard_normal(64).astype(np.float32)
    x[5] = -np.inf
    mx = np.zeros(64, np.float32)
    sm = np.zeros(64, np.float32)
    fp = ctypes.POINTER(ctypes.c_float)
    assert kat.kat_pair(x.ctypes.data_as(fp), mx.ctypes.data_as(fp), sm.ctypes.data_as(fp)) == 0
    partner = x[np.arange(64) ^ 32]
    assert np.array_equal(mx, np.maximum(x, partner))
    assert np.array_equal(sm, (x + partner).astype(np.float32))


def test_dma_lane_placement(kat):
    """dma_16b: lane i's 16 bytes from its own source offset land at LDS
    base + 16*i; nothing outside the 1 KiB window is touched."""
    print("case global_load_lds_dwordx4 placement", flush=True)
    out = np.zeros(512, np.int32)
    assert kat.kat_dma(out.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))) == 0
    assert np.all(out[:256] == -1)
    lanes = np.arange(64)
    src_chunk = (lanes * 7) % 64
    expect = (src_chunk[:, None] * 4 + np.arange(4)[None, :]).reshape(-1)
    assert np.array_equal(out[256:], expect)


@pytest.mark.parametrize("total", [1, 5, 8, 9, 15, 16, 17, 100, 2048, 4097, 12345])
def test_xcd_remap_is_contiguous_per_xcd(kat, total):
    """xcd_remap is a permutation of [0, total) under which the dispatch
    indices the hardware sends to XCD x (b % 8 == x) own one contiguous
    logical range, the ranges ascending with x."""
    print(f"case xcd_remap total={total}", flush=True)
    out = np.zeros(total, np.int32)
    assert kat.kat_xcd_remap(total, out.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))) == 0
    assert np.array_equal(np.sort(out), np.arange(total))
    prev_hi = -1
    for x in range(8):
        ids = np.sort(out[np.arange(total) % 8 == x])
        if ids.size == 0:
            continue
        assert np.array_equal(ids, np.arange(ids[0], ids[0] + ids.size)), x
        assert ids[0] == prev_hi + 1
        prev_hi = ids[-1]
        # consecutive dispatches on one XCD walk its range in order
        assert np.all(np.diff(out[np.arange(total) % 8 == x]) == 1)


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
def test_row_sum_mfma_lane_map(kat, dtype):
    """row_sum_mfma: the 16x16x32 MFMA with the selector operand sums each
    query row's keys of a P^T chunk (lane l: row l % 32, key half l / 32),
    row_sum_scale multiplies each row's running sum by that row's factor,
    and row_sum_of_lane hands every lane its row's total.  Values k/64 with
    k < 256 are exact in both types, so the sums are exact."""
    print(f"case row_sum_mfma {dtype}", flush=True)
    rng = np.random.default_rng(9)
    vals = rng.integers(0, 256, size=(2, 64, 8)).astype(np.float32) / 64.0
    if dtype == "fp16":
        bits = np.ascontiguousarray(vals.astype(np.float16).view(np.uint16))
    else:
        bits = np.ascontiguousarray((vals.view(np.uint32) >> 16).astype(np.uint16))
    row_f = rng.integers(1, 9, size=32).astype(np.float32) / 8.0   # exact factors
    f = np.concatenate([row_f, row_f]).astype(np.float32)
    out = np.zeros(64, np.float32)
    u16p = ctypes.POINTER(ctypes.c_uint16)
    fp = ctypes.POINTER(ctypes.c_float)
    assert kat.kat_row_sum(bits.ctypes.data_as(u16p), f.ctypes.data_as(fp),
                           1 if dtype == "bf16" else 0, out.ctypes.data_as(fp)) == 0
    lane_sums = vals.astype(np.float64).sum(axis=2)           # [chunk, lane]
    row_sums = lane_sums[:, :32] + lane_sums[:, 32:]          # [chunk, row]: both key halves
    rows = row_sums[0] * row_f + row_sums[1]
    expect = np.concatenate([rows, rows])
    assert np.array_equal(out, expect.astype(np.float32)), (out[:8], expect[:8])
