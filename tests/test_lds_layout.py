"""CPU checks of the K/V tile layout in LDS (flash-attention_amd/csrc/
fa_lds_layout.h), on a host build of the same functions the kernel runs
(tests/lds/fa_lds_map.cpp, compiled here with g++).

For D in {64, 128} and workgroups of 4 and 8 waves:
- the staging DMA covers every (key, 16-byte chunk) of a tile exactly once
  (a bijection onto the tile's bytes);
- every K operand read (ds_read_b128, A operand of S^T = K Q^T) and every V^T
  operand read (ds_read_b64_tr_b16) finds the bytes the DMA put there for
  the key and head dims the MFMA lane maps require;
- the offsets the kernel uses for key block 1 and for later V chunks/halves
  (a constant added to block 0 / chunk 0) equal the general formula;
- no access has a bank conflict, under this model of the gfx950 LDS: 64
  banks of 4 bytes; ds_read_b128 serves 16 lanes (256 bytes) per cycle,
  ds_read_b64_tr_b16 32 lanes, and ds_write_b128 8 lanes (128 bytes), whose
  addresses conflict when they agree mod 128 bytes; within a cycle, distinct
  dwords on one bank are served one after the other.  The model is
  calibrated on the hardware: it reproduces the conflict cycles that
  tests/lds/lds_bank_probe.hip measured for 31 access patterns
  (profiles/lds_bank_probe.md), and the 65536 cycles per C2 launch of the
  previous 128-byte row swizzle;
- the bank check sees a dropped swizzle bit: a copy built with one bit of the
  K or V swizzle cleared still reads what it wrote, but conflicts;
- the same four checks for the layout of the 16x16x32 kernel (lds::Tile16,
  dma_slot16, k16_read_offset, v16_read_offset: its K reads cover 16 keys x
  one chunk per 16-lane group, its V^T reads 8 keys x 32 bytes per 32-lane
  pass), against that kernel's MFMA lane maps;
- the row tiles a wave stages on its own (Q operands, the O and split-partial
  stores) are bijections whose 16-byte writes and reads are conflict free, a
  copy with a row-swizzle bit cleared conflicts, and 8-byte writes would
  conflict under the dword-pass model the hardware counter supports.

Reference counterpart: the swizzle offset known-answer tests of
tests/unit/layout/test_tile_to_shape_runtime.cu:152-168 (for the NVIDIA
Swizzle<3,3,3> layout, which this build does not use).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(HERE)
CSRC = os.path.join(REPO, "flash-attention_amd", "csrc")
SRC = os.path.join(HERE, "lds", "fa_lds_map.cpp")

BANKS, BANK_BYTES = 64, 4


def _build(out_dir, defines=()):
    out = os.path.join(out_dir, "libfa_lds_map_%d.so" % abs(hash(defines)))
    cmd = ["g++", "-O1", "-std=c++17", "-shared", "-fPIC", "-I", CSRC,
           *[f"-D{d}" for d in defines], SRC, "-o", out]
    subprocess.run(cmd, check=True)
    lib = ctypes.CDLL(out)
    ip = ctypes.POINTER(ctypes.c_int)
    lib.fa_lds_dma_map.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ip, ip]
    lib.fa_lds_k_reads.argtypes = [ctypes.c_int, ip]
    lib.fa_lds_v_reads.argtypes = [ctypes.c_int, ip]
    lib.fa_lds_dma_map16.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ip, ip]
    lib.fa_lds_k16_reads.argtypes = [ctypes.c_int, ip]
    lib.fa_lds_v16_reads.argtypes = [ctypes.c_int, ip]
    return lib


@pytest.fixture(scope="module")
def lib(tmp_path_factory):
    return _build(str(tmp_path_factory.mktemp("lds")))


def _ptr(a):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_int))


def _dma_slots(lib, D, NW, is_v):
    """slot[key, chunk] = LDS byte offset (within the tile) the DMA writes it
    to.  A DMA lane's destination is fixed by the instruction: byte
    (wave*ITERS + it)*1024 + 16*lane of the tile, in the map's order."""
    rowb = 2 * D
    n = 64 * rowb // 16
    r = np.empty(n, np.int32)
    c = np.empty(n, np.int32)
    assert lib.fa_lds_dma_map(D, NW, int(is_v), _ptr(r), _ptr(c)) == n
    slot = np.full((64, rowb // 16), -1, np.int64)
    dest = np.arange(n, dtype=np.int64) * 16
    assert ((r >= 0) & (r < 64) & (c >= 0) & (c < rowb // 16)).all()
    slot[r, c] = dest
    return slot, r, c


def _k_reads(lib, D):
    ks = D // 16
    off = np.empty(2 * ks * 64, np.int32)
    assert lib.fa_lds_k_reads(D, _ptr(off)) == off.size
    return off.reshape(2, ks, 64).astype(np.int64)


def _v_reads(lib, D):
    nd = D // 32
    off = np.empty(4 * 2 * nd * 64, np.int32)
    assert lib.fa_lds_v_reads(D, _ptr(off)) == off.size
    return off.reshape(4, 2, nd, 64).astype(np.int64)


def _conflict_cycles(addrs, nbytes, lanes_per_cycle, window):
    """Bank-conflict cycles of one wave-wide LDS instruction, the quantity
    SQ_LDS_BANK_CONFLICT counts: the lanes are served `lanes_per_cycle` at a
    time in lane order, each touching `nbytes` bytes from its address; within
    one cycle, distinct dwords whose addresses agree mod `window` bytes share
    a bank and are served one after the other, so a cycle whose fullest bank
    holds k distinct dwords costs k - 1 extra cycles."""
    nbanks = window // BANK_BYTES
    total = 0
    for g0 in range(0, len(addrs), lanes_per_cycle):
        seen = {}
        for a in addrs[g0:g0 + lanes_per_cycle]:
            for w in range(0, nbytes, BANK_BYTES):
                word = (int(a) + w) // BANK_BYTES
                seen.setdefault(word % nbanks, set()).add(word)
        total += max(len(s) for s in seen.values()) - 1
    return total


# The instruction forms, as measured on the MI355X by tests/lds/lds_bank_probe.hip
# (kPatterns below): ds_read_b128 serves 16 lanes (256 bytes) per cycle over
# all 64 banks; ds_write_b128 serves 8 lanes (128 bytes) per cycle, and two of
# them conflict when their addresses agree mod 128 bytes; ds_read_b64_tr_b16
# serves 32 lanes (256 bytes) per cycle.
def read128(addrs):
    return _conflict_cycles(addrs, 16, 16, 256)


def write128(addrs):
    return _conflict_cycles(addrs, 16, 8, 128)


def read_tr64(addrs):
    return _conflict_cycles(addrs, 8, 32, 256)


CASES = [(D, NW) for D in (64, 128) for NW in (4, 8)]


@pytest.mark.parametrize("D,NW", CASES)
@pytest.mark.parametrize("is_v", [False, True], ids=["K", "V"])
def test_dma_is_a_bijection_onto_the_tile(lib, D, NW, is_v):
    slot, r, c = _dma_slots(lib, D, NW, is_v)
    assert (slot >= 0).all(), "some (key, chunk) is never staged"
    pairs = r.astype(np.int64) * (2 * D // 16) + c
    assert np.unique(pairs).size == pairs.size, "some (key, chunk) is staged twice"


@pytest.mark.parametrize("D,NW", CASES)
def test_k_reads_find_the_staged_keys(lib, D, NW):
    slot, _, _ = _dma_slots(lib, D, NW, False)
    off = _k_reads(lib, D)
    lane = np.arange(64)
    for kb in range(2):
        for kk in range(D // 16):
            # 32x32x16 A operand: lane l supplies row l % 32 (the key) and
            # k-elements 8(l / 32) .. +7 of k-step kk (head dims 16kk + ...).
            key = kb * 32 + lane % 32
            chunk = 2 * kk + lane // 32
            assert np.array_equal(off[kb, kk], slot[key, chunk]), (kb, kk)
    # the kernel's form: block 1 = block 0 + 32 rows
    assert np.array_equal(off[1], off[0] + 32 * 2 * D)


@pytest.mark.parametrize("D,NW", CASES)
def test_v_reads_find_the_staged_keys(lib, D, NW):
    slot, _, _ = _dma_slots(lib, D, NW, True)
    off = _v_reads(lib, D)
    lane = np.arange(64)
    lj, hg, g = lane % 16, (lane // 16) % 2, lane // 32
    for ch in range(4):
        for hf in range(2):
            for db in range(D // 32):
                key = 16 * ch + 8 * hf + 4 * g + lj // 4
                col = 32 * db + 16 * hg + 4 * (lj % 4)
                want = slot[key, col // 8] + (col % 8) * 2
                assert np.array_equal(off[ch, hf, db], want), (ch, hf, db)
                # the kernel's form: chunk/half offsets added as immediates
                assert np.array_equal(off[ch, hf, db], off[0, 0, db] + (16 * ch + 8 * hf) * 2 * D)


def _read_conflicts(lib, D):
    k = _k_reads(lib, D)
    v = _v_reads(lib, D)
    kc = sum(read128(k[kb, kk]) for kb in range(2) for kk in range(D // 16))
    vc = sum(read_tr64(v[ch, hf, db]) for ch in range(4) for hf in range(2) for db in range(D // 32))
    return kc, vc


@pytest.mark.parametrize("D", [64, 128])
def test_reads_are_bank_conflict_free(lib, D):
    assert _read_conflicts(lib, D) == (0, 0)


def test_dma_writes_are_bank_conflict_free():
    # each DMA instruction writes 64 lanes x 16 contiguous bytes
    assert write128(np.arange(64) * 16) == 0


@pytest.mark.parametrize("D,k_clear,v_clear", [(128, 8, 0), (128, 1, 0), (128, 0, 4),
                                               (128, 0, 8), (64, 4, 0), (64, 1, 0),
                                               (64, 0, 4)])
def test_dropped_swizzle_bit_is_detected(tmp_path, D, k_clear, v_clear):
    """One swizzle bit cleared: reads still find what the DMA wrote (both
    sides share the swizzle), but the bank check reports conflicts."""
    mut = _build(str(tmp_path), (f"FA_LDS_SWZ_K_CLEAR={k_clear}", f"FA_LDS_SWZ_V_CLEAR={v_clear}"))
    slot, _, _ = _dma_slots(mut, D, 4, False)
    off = _k_reads(mut, D)
    lane = np.arange(64)
    assert np.array_equal(off[0, 0], slot[lane % 32, lane // 32])
    kc, vc = _read_conflicts(mut, D)
    if k_clear:
        assert kc > 0, "a dropped K swizzle bit went unnoticed"
    if v_clear:
        assert vc > 0, "a dropped V swizzle bit went unnoticed"


# ---- the 16x16x32 kernel's layout (lds::Tile16) ----

def _dma_slots16(lib, D, NW, is_v):
    rowb = 2 * D
    n = 64 * rowb // 16
    r = np.empty(n, np.int32)
    c = np.empty(n, np.int32)
    assert lib.fa_lds_dma_map16(D, NW, int(is_v), _ptr(r), _ptr(c)) == n
    slot = np.full((64, rowb // 16), -1, np.int64)
    slot[r, c] = np.arange(n, dtype=np.int64) * 16
    return slot, r, c


def _k16_reads(lib, D):
    off = np.empty(4 * (D // 32) * 64, np.int32)
    assert lib.fa_lds_k16_reads(D, _ptr(off)) == off.size
    return off.reshape(4, D // 32, 64).astype(np.int64)


def _v16_reads(lib, D):
    off = np.empty(2 * 2 * (D // 16) * 64, np.int32)
    assert lib.fa_lds_v16_reads(D, _ptr(off)) == off.size
    return off.reshape(2, 2, D // 16, 64).astype(np.int64)


@pytest.mark.parametrize("D,NW", CASES)
@pytest.mark.parametrize("is_v", [False, True], ids=["K", "V"])
def test_dma16_is_a_bijection_onto_the_tile(lib, D, NW, is_v):
    slot, r, c = _dma_slots16(lib, D, NW, is_v)
    assert (slot >= 0).all()
    pairs = r.astype(np.int64) * (2 * D // 16) + c
    assert np.unique(pairs).size == pairs.size


@pytest.mark.parametrize("D,NW", CASES)
def test_k16_reads_find_the_staged_keys(lib, D, NW):
    slot, _, _ = _dma_slots16(lib, D, NW, False)
    off = _k16_reads(lib, D)
    lane = np.arange(64)
    for kb in range(4):
        for st in range(D // 32):
            # 16x16x32 A operand: lane l supplies row l % 16 (the key) and
            # k-elements 8(l / 16) .. +7 of k-step st (head dims 32st + ...).
            want = slot[16 * kb + lane % 16, 4 * st + lane // 16]
            assert np.array_equal(off[kb, st], want), (kb, st)
            # the kernel's form: key block kb = block 0 + 16kb rows
            assert np.array_equal(off[kb, st], off[0, st] + 16 * kb * 2 * D)


@pytest.mark.parametrize("D,NW", CASES)
def test_v16_reads_find_the_staged_keys(lib, D, NW):
    """Each 16-lane group g of a transposing read hands lane i element i % 4 of
    the words addressed by lanes 4e + i / 4 (e = 0..3), so lane i must receive
    V[32ch + 16h + 4g + e][16db + i]: the word of lane 4e + q holds row
    32ch + 16h + 4g + e, columns 16db + 4q .. +3."""
    slot, _, _ = _dma_slots16(lib, D, NW, True)
    off = _v16_reads(lib, D)
    lane = np.arange(64)
    l16, g = lane % 16, lane // 16
    for ch in range(2):
        for h in range(2):
            for db in range(D // 16):
                key = 32 * ch + 16 * h + 4 * g + l16 // 4
                col = 16 * db + 4 * (l16 % 4)
                want = slot[key, col // 8] + (col % 8) * 2
                assert np.array_equal(off[ch, h, db], want), (ch, h, db)
                assert np.array_equal(off[ch, h, db], off[0, 0, db] + (32 * ch + 16 * h) * 2 * D)
                # what the receiving lanes get: lane i of group gg, element e
                for gg in range(4):
                    for i in range(16):
                        for e in range(4):
                            src = 16 * gg + 4 * e + i // 4  # the addressing lane
                            got = off[ch, h, db][src] + (i % 4) * 2
                            k_, c_ = 32 * ch + 16 * h + 4 * gg + e, 16 * db + i
                            assert got == slot[k_, c_ // 8] + (c_ % 8) * 2, (ch, h, db, gg, i, e)


def _read_conflicts16(lib, D):
    k = _k16_reads(lib, D)
    v = _v16_reads(lib, D)
    kc = sum(read128(k[kb, st]) for kb in range(4) for st in range(D // 32))
    vc = sum(read_tr64(v[ch, h, db]) for ch in range(2) for h in range(2) for db in range(D // 16))
    return kc, vc


@pytest.mark.parametrize("D", [64, 128])
def test_reads16_are_bank_conflict_free(lib, D):
    assert _read_conflicts16(lib, D) == (0, 0)


@pytest.mark.parametrize("D,v_clear", [(128, 2), (128, 4), (128, 8), (64, 2), (64, 4)])
def test_dropped_v16_swizzle_bit_is_detected(tmp_path, D, v_clear):
    """A 16x16 V swizzle bit cleared: the reads still find what the DMA wrote,
    but the 32-lane passes conflict."""
    mut = _build(str(tmp_path), (f"FA_LDS_SWZ_V16_CLEAR={v_clear}",))
    slot, _, _ = _dma_slots16(mut, D, 4, True)
    off = _v16_reads(mut, D)
    lane = np.arange(64)
    l16, g = lane % 16, lane // 16
    key = 4 * g + l16 // 4
    col = 4 * (l16 % 4)
    assert np.array_equal(off[0, 0, 0], slot[key, col // 8] + (col % 8) * 2)
    assert _read_conflicts16(mut, D)[1] > 0, "a dropped V16 swizzle bit went unnoticed"


# ---- row tiles (lds::row_tile_offset) ----
# A wave stages 32 rows of `rowb` bytes on its own: Q (rowb = 2D, 4-wave
# workgroups) for its B operands, and on the way out O (rowb = 2D) or the
# fp32 split partials (rowb = 128 x head-dim blocks per pass).  Every write
# and read is 16 bytes per lane.

def _row_lib(lib):
    lib.fa_lds_row_offset.argtypes = [ctypes.c_int] * 3
    return lib


def _row_off(lib, r, c, rowb):
    return lib.fa_lds_row_offset(int(r), int(c), rowb)


@pytest.mark.parametrize("rowb", [128, 256, 512])
def test_row_tile_is_a_bijection(lib, rowb):
    _row_lib(lib)
    nc = rowb // 16
    offs = sorted(_row_off(lib, r, c, rowb) for r in range(32) for c in range(nc))
    assert offs == list(range(0, 32 * rowb, 16))


def _chunk_writes(lib, rowb):
    """The output writes: ds_write_b128, lane (l32, g) writes chunk 2p + g of
    row l32 (O after the lane-pair swap; the split partials directly)."""
    return [[_row_off(lib, l % 32, 2 * p + l // 32, rowb) for l in range(64)]
            for p in range(rowb // 32)]


def _row_reads(lib, rowb):
    """Whole-row reads: ds_read_b128, lane i reads chunk i % nc of row
    j * (64 / nc) + i / nc."""
    nc = rowb // 16
    rpi = 64 // nc
    return [[_row_off(lib, j * rpi + l // nc, l % nc, rowb) for l in range(64)]
            for j in range(32 // rpi)]


def _q_operand_reads(lib, rowb):
    """Q B-operand reads: ds_read_b128, lane (l32, g) reads chunk 2kk + g of
    row l32."""
    return [[_row_off(lib, l % 32, 2 * kk + l // 32, rowb) for l in range(64)]
            for kk in range(rowb // 32)]


def _row_conflicts(lib, rowb):
    return {
        "writes": sum(write128(a) for a in _chunk_writes(lib, rowb)),
        "row_reads": sum(read128(a) for a in _row_reads(lib, rowb)),
        "q_reads": sum(read128(a) for a in _q_operand_reads(lib, rowb)),
    }


@pytest.mark.parametrize("rowb", [128, 256, 512])
def test_row_tile_accesses_are_bank_conflict_free(lib, rowb):
    _row_lib(lib)
    assert _row_conflicts(lib, rowb) == {"writes": 0, "row_reads": 0, "q_reads": 0}


def _dword_pass_conflicts(addrs):
    """8-byte plain accesses, served one dword at a time across all 64 lanes
    (the model that matches the hardware counter: SQ_LDS_BANK_CONFLICT was
    1048576 per C3 launch with 8-byte O-staging writes, whatever the swizzle,
    and 0 with the 16-byte ones)."""
    return sum(_conflict_cycles([a + 4 * d for a in addrs], 4, 64, 256) for d in range(2))


@pytest.mark.parametrize("rowb", [128, 256])
def test_eight_byte_output_writes_would_conflict(lib, rowb):
    """Why O is swapped into 16-byte chunks first: writing each lane's 8-byte
    half chunk (cols 8c + 4g .. +3 of row l32) directly puts every low dword
    on an even bank, a 2-way conflict under any row swizzle."""
    _row_lib(lib)
    for c in range(rowb // 16):
        halves = [_row_off(lib, l % 32, c, rowb) + 8 * (l // 32) for l in range(64)]
        assert _dword_pass_conflicts(halves) > 0
    assert all(_dword_pass_conflicts([a + 8 * (l // 32) for l, a in enumerate(w)]) > 0
               for w in _chunk_writes(lib, rowb))


@pytest.mark.parametrize("rowb,clear,which", [
    (256, 8, "q_reads"),
    (256, 1, "writes"),
    (128, 4, "writes"),
    (128, 1, "writes"),
    (128, 2, "q_reads"),
    (512, 4, "writes"),
])
def test_dropped_row_swizzle_is_detected(tmp_path, rowb, clear, which):
    """With one row-swizzle bit cleared the tile is still a bijection but the
    named accesses conflict."""
    mut = _row_lib(_build(str(tmp_path), (f"FA_LDS_ROW_SWZ_CLEAR={clear}",)))
    nc = rowb // 16
    offs = sorted(_row_off(mut, r, c, rowb) for r in range(32) for c in range(nc))
    assert offs == list(range(0, 32 * rowb, 16))
    assert _row_conflicts(mut, rowb)[which] > 0


# ---- calibration of the bank model on the hardware ----
# tests/lds/lds_bank_probe.hip runs each pattern below as its own dispatch
# (64 instructions per wave, 1024 waves) and profiles/lds_bank_probe.md holds
# SQ_LDS_BANK_CONFLICT / SQ_INSTS_LDS for each: the conflict cycles of one
# instruction.  The model must give the same number for every pattern.

def _old_row128(r, c):
    """The row tile of 128-byte rows before the current swizzle (chunk c of
    row r at c ^ ((r >> 1) & 7)), which the C2 counters were measured with."""
    return r * 128 + ((c ^ ((r >> 1) & 7)) << 4)


def _probe_patterns(lib):
    """(instruction form, 64 lane offsets) of each probe pattern, in the
    probe's order (its offset_of<P>)."""
    _row_lib(lib)
    lane = np.arange(64)
    l32, g = lane % 32, lane // 32
    k64, k128 = _k_reads(lib, 64), _k_reads(lib, 128)
    v64, v128 = _v_reads(lib, 64), _v_reads(lib, 128)
    row = lambda rs, cs, rowb: [_row_off(lib, r, c, rowb) for r, c in zip(rs, cs)]
    return [
        (read128, lane * 16),
        (read128, lane * 256),
        (write128, [_old_row128(r, 0 + q) for r, q in zip(l32, g)]),
        (write128, [_old_row128(r, 2 + q) for r, q in zip(l32, g)]),
        (write128, [_old_row128(r, 4 + q) for r, q in zip(l32, g)]),
        (write128, [_old_row128(r, 6 + q) for r, q in zip(l32, g)]),
        (read128, [_old_row128(l // 8, l % 8) for l in lane]),
        (read128, [_old_row128(8 + l // 8, l % 8) for l in lane]),
        (read128, [_old_row128(r, 0 + q) for r, q in zip(l32, g)]),
        (read128, [_old_row128(r, 2 + q) for r, q in zip(l32, g)]),
        (write128, row(l32, g, 256)),
        (read128, row(lane // 16, lane % 16, 256)),
        (read128, k64[0, 0]),
        (read128, k64[0, 1]),
        (read_tr64, v64[0, 0, 0]),
        (read_tr64, v64[0, 0, 1]),
        (write128, lane * 16),
        (write128, lane * 256),
        (read128, k128[0, 0]),
        (read_tr64, v128[0, 0, 0]),
        (write128, row(l32, 2 + g, 256)),
        (read128, row(l32, g, 256)),
        (write128, (lane % 16) * 16 + (lane // 16) * 1024),
        (write128, l32 * 16 + g * 8192),
        (read128, l32 * 16 + g * 8192),
        (write128, (lane % 8) * 16 + ((lane // 8) % 2) * 8192 + (lane // 16) * 128),
        (write128, row(l32, g, 128)),
        (write128, row(l32, 6 + g, 128)),
        (read128, row(lane // 8, lane % 8, 128)),
        (read128, row(l32, g, 128)),
        (read128, row(l32, 6 + g, 128)),
    ]


# Conflict cycles per instruction measured by the probe (MI355X, ROCm 7.2).
MEASURED_CONFLICT_CYCLES = [0, 60, 8, 8, 8, 8, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0,
                            0, 56, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0]


def test_bank_model_matches_the_probe(lib):
    """The model reproduces the measured conflict cycles of every probe
    pattern: the 16-lane, 256-byte read cycles (60 cycles when 16 lanes share
    a bank group), the 8-lane, 128-byte write cycles (56 when 8 lanes share
    one; 8 for the old 128-byte row tile, whose rows 2i and 2i + 1 agree mod
    128 bytes although they differ mod 256), and zero elsewhere."""
    pats = _probe_patterns(lib)
    assert len(pats) == len(MEASURED_CONFLICT_CYCLES)
    got = [form(np.asarray(addrs, np.int64)) for form, addrs in pats]
    assert got == MEASURED_CONFLICT_CYCLES


def test_bank_model_predicts_the_c2_count(lib):
    """C2 (B4 H16 N1024 D64 fp16: 512 workgroups of 4 waves) counted
    SQ_LDS_BANK_CONFLICT = 65536 per launch with the old 128-byte row
    swizzle.  Under the model every read of that kernel is conflict-free and
    each of a wave's 4 O-staging writes costs 8 cycles: 2048 waves x 32 =
    65536.  The current swizzle gives 0."""
    _row_lib(lib)
    k, v = _k_reads(lib, 64), _v_reads(lib, 64)
    tiles = 1024 // 64
    reads = tiles * (sum(read128(k[kb, kk]) for kb in range(2) for kk in range(4)) +
                     sum(read_tr64(v[ch, hf, db]) for ch in range(4) for hf in range(2)
                         for db in range(2)))
    lane = np.arange(64)
    old_writes = sum(write128([_old_row128(l % 32, 2 * p + l // 32) for l in lane]) for p in range(4))
    old_reads = sum(read128([_old_row128(j * 8 + l // 8, l % 8) for l in lane]) for j in range(4))
    old_q = sum(read128([_old_row128(l % 32, 2 * kk + l // 32) for l in lane]) for kk in range(4))
    waves = 4 * 16 * (1024 // 128) * 4
    assert waves * (reads + old_writes + old_reads + old_q) == 65536
    now = _row_conflicts(lib, 128)
    assert waves * (reads + now["writes"] + now["row_reads"] + now["q_reads"]) == 0
