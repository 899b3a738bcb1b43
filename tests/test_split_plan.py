"""CPU tests of the split-KV work plan (fa_fwd_plan in include/fa_mi355x.h).

The plan decides, on the host, whether a problem's key ranges are split
across workgroups and how.  The kernel trusts it completely: every key tile
of every q-tile must be computed by exactly one work item, every split q-tile
needs its own run of partial slots, and the workspace must hold them all.
These are the invariants checked here, over the BASELINE configurations and
a sweep of shapes, for the MI355X's 256 CUs and other CU counts.  Nothing
here touches a GPU.
"""
from __future__ import annotations

import ctypes

import pytest

import abi_ctypes as A
from test_abi import contiguous

BN = 64  # keys per tile


@pytest.fixture(scope="module")
def lib():
    return A.load()


def plan(lib, p, cus=256):
    out = A.FaFwdPlan()
    rc = lib.fa_fwd_plan(ctypes.byref(p), cus, ctypes.byref(out))
    assert rc == A.FA_OK, lib.fa_last_error().decode()
    return out


def tiles(qb, N, BM, causal):
    kv = min(N, (qb + 1) * BM) if causal else N
    return (kv + BN - 1) // BN


def check_table(pl, B, H, N, D, causal, cus=256):
    """XCD placement table: one XCD's work items (every q-tile of its heads,
    none split), each (head, q-tile) exactly once; the longest items run
    alone and the shared CUs pair long with short; no workspace."""
    BM = pl.block_rows
    nq = (N + BM - 1) // BM
    hpx, cpx = B * H // 8, cus // 8
    n = pl.n_items
    assert causal and BM == 128 and B * H == 8 * pl.xcd_heads == 8 * hpx
    assert cpx < hpx * nq and n <= 2 * cpx
    assert pl.key_halves == 1
    assert n == hpx * nq and pl.n_merge == 0 and pl.n_slots == 0 and pl.workspace_bytes == 0
    seen = set()
    for i in range(n):
        assert pl.n_chunks[i] == 1 and pl.slot[i] == -1
        assert pl.tile_begin[i] == 0 and pl.tile_end[i] == tiles(pl.q_tile[i], N, BM, causal)
        seen.add((pl.head[i], pl.q_tile[i]))
    assert sorted(seen) == [(h, q) for h in range(hpx) for q in range(nq)]
    lens = [pl.tile_end[i] - pl.tile_begin[i] for i in range(n)]
    m = max(n - cpx, 0)
    alone = lens[m:cpx]
    shared = [(lens[j], lens[cpx + j]) for j in range(m)]
    if alone and shared:
        assert min(alone) >= max(max(a, b) for a, b in shared)
    firsts = [a for a, _ in shared]
    seconds = [b for _, b in shared]
    assert firsts == sorted(firsts, reverse=True) and seconds == sorted(seconds)
    if shared:
        assert min(firsts) >= max(seconds)


def check_pair(pl, B, H, N, causal, cus=256):
    """Pair mode: causal, 128-row q-tiles, 0.75 to 2 of them per CU, one
    workgroup per q-tile (no items, no workspace)."""
    items = B * H * ((N + 127) // 128)
    assert causal and pl.block_rows == 128 and pl.key_halves == 2
    assert 4 * items >= 3 * cus and items < 2 * cus
    assert pl.n_items == 0 and pl.xcd_heads == 0 and pl.workspace_bytes == 0


def check_plan(pl, B, H, N, D, causal):
    BM = pl.block_rows
    nq = (N + BM - 1) // BM
    n = pl.n_items
    assert 0 < n <= A.FA_PLAN_MAX_ITEMS
    items = [(pl.q_tile[i], pl.tile_begin[i], pl.tile_end[i], pl.n_chunks[i], pl.slot[i])
             for i in range(n)]
    # every key tile of every q-tile exactly once, chunks non-empty
    by_q = {}
    for qb, tb, te, nch, slot in items:
        assert 0 <= qb < nq
        assert 0 <= tb < te <= tiles(qb, N, BM, causal)
        by_q.setdefault(qb, []).append((tb, te, nch, slot))
    assert sorted(by_q) == list(range(nq))
    slots_used = []
    merged = 0
    for qb, chunks in by_q.items():
        chunks.sort()
        nch = chunks[0][2]
        assert all(c[2] == nch for c in chunks) and len(chunks) == nch <= 255
        assert chunks[0][0] == 0 and chunks[-1][1] == tiles(qb, N, BM, causal)
        for a, b in zip(chunks, chunks[1:]):
            assert a[1] == b[0]
        if nch == 1:
            assert chunks[0][3] == -1
        else:
            merged += 1
            s = [c[3] for c in chunks]
            assert s == list(range(s[0], s[0] + nch))  # a run of consecutive slots
            slots_used += s
    assert merged == pl.n_merge > 0
    assert sorted(slots_used) == list(range(pl.n_slots))  # disjoint, dense
    # dispatch order: longest first
    lens = [te - tb for _, tb, te, _, _ in items]
    assert lens == sorted(lens, reverse=True)
    assert pl.workspace_bytes == B * H * pl.n_slots * BM * (D * 4 + 16)
    # the split shortens the longest work item
    assert max(lens) < max(tiles(qb, N, BM, causal) for qb in range(nq))


@pytest.mark.parametrize("name,B,H,N,D,causal,dtype,split", [
    ("C1", 1, 1, 128, 128, 0, A.FA_DTYPE_F16, False),
    ("C2", 4, 16, 1024, 64, 0, A.FA_DTYPE_F16, False),
    ("C3", 4, 32, 4096, 128, 0, A.FA_DTYPE_F16, False),
    ("C4", 2, 32, 8192, 128, 1, A.FA_DTYPE_BF16, False),
    ("C5", 1, 16, 16384, 128, 1, A.FA_DTYPE_F16, False),
    ("C5r", 1, 16, 3000, 128, 1, A.FA_DTYPE_F16, "pair"),
    ("C5r/2", 1, 8, 3000, 128, 1, A.FA_DTYPE_F16, "pair"),
    ("C5r/4", 1, 4, 3000, 128, 1, A.FA_DTYPE_F16, True),
])
def test_baseline_configs(lib, name, B, H, N, D, causal, dtype, split):
    """The BASELINE configurations run unsplit: C2-C5 fill the machine; C5r
    (384 q-tiles of 128 rows on 256 CUs) runs in pair mode, and so does the
    same shape with half its heads (192 = 0.75 per CU).  With a quarter of
    its heads (96 q-tiles) the plan splits the long q-tiles instead."""
    p = contiguous(B=B, H=H, N=N, D=D, dtype=dtype, causal=causal)
    pl = plan(lib, p)
    assert pl.block_rows == (256 if (N >= 2048 and not causal) or
                             (causal and dtype == A.FA_DTYPE_F16 and N >= 8192) else 128)
    if split == "pair":
        check_pair(pl, B, H, N, causal)
    elif not split:
        assert pl.n_items == 0 and pl.workspace_bytes == 0 and pl.n_slots == 0
        assert pl.key_halves == 1
    else:
        assert pl.xcd_heads == 0
        check_plan(pl, B, H, N, D, causal)


@pytest.mark.parametrize("B,H,N,dtype,causal,cus,group", [
    (2, 32, 8192, A.FA_DTYPE_BF16, 1, 256, 2),   # C4: 8 heads per XCD, 64 q-tiles each
    (2, 32, 8192, A.FA_DTYPE_BF16, 1, 304, 4),   # 38 CUs per XCD: a pair is under 2 rounds
    (4, 32, 4096, A.FA_DTYPE_F16, 1, 256, 4),    # 32 q-tiles per head: 4 heads for 2 rounds
    (8, 32, 1024, A.FA_DTYPE_F16, 1, 256, 4),
    (1, 16, 16384, A.FA_DTYPE_F16, 1, 256, 2),   # C5: 2 heads per XCD, 8-wave
    (2, 8, 8192, A.FA_DTYPE_BF16, 1, 256, 2),
    (1, 24, 8192, A.FA_DTYPE_F16, 1, 256, 3),    # 3 heads per XCD: one group
    (1, 16, 3000, A.FA_DTYPE_F16, 1, 256, 2),    # C5r, pair mode
    (1, 12, 4096, A.FA_DTYPE_F16, 1, 256, 0),    # B*H not a multiple of 8
    (4, 32, 4096, A.FA_DTYPE_F16, 0, 256, 0),    # non-causal
    (1, 16, 4096, A.FA_DTYPE_F16, 1, 256, 0),    # XCD placement table
    (1, 4, 3000, A.FA_DTYPE_F16, 1, 256, 0),     # split-KV
])
def test_causal_head_group(lib, B, H, N, dtype, causal, cus, group):
    """Causal grids in plain order (no items) with B*H a multiple of 8 run
    each XCD's heads in groups: 4 when the XCD's head count is a multiple of
    4, else all of them, and 2 when a group of 2 heads still fills the XCD's
    workgroup slots (two per CU for 128-row q-tiles, one otherwise) twice.
    The group always divides the XCD's head count."""
    p = contiguous(B=B, H=H, N=N, D=128, dtype=dtype, causal=causal)
    pl = plan(lib, p, cus)
    assert pl.head_group == group and pl.reserved == 0
    if group:
        assert pl.n_items == 0 and (B * H // 8) % group == 0


def test_pair_mode_range(lib):
    """Pair mode covers causal grids of 0.75 to 2 q-tiles (128 rows) per CU,
    whatever the CU count: C5r's 384 q-tiles are in range on 256 and 512 CUs,
    too many on 128 (plain 4-wave grid) and too few on 1024 (split-KV)."""
    p = contiguous(B=1, H=16, N=3000, D=128, causal=1)
    for cus in (256, 512):
        check_pair(plan(lib, p, cus=cus), 1, 16, 3000, 1, cus)
    small = plan(lib, p, cus=128)
    assert small.key_halves == 1 and small.n_items == 0 and small.workspace_bytes == 0
    big = plan(lib, p, cus=1024)
    assert big.key_halves == 1
    check_plan(big, 1, 16, 3000, 128, 1)
    # non-causal and 8-wave causal problems never pair
    for q in (contiguous(B=1, H=16, N=3000, D=128, causal=0),
              contiguous(B=1, H=1, N=16384, D=128, causal=1)):
        assert plan(lib, q).key_halves == 1


@pytest.mark.parametrize("B,H,N,D,dtype", [
    (4, 16, 1000, 64, A.FA_DTYPE_BF16),   # C2c's shape: 8 heads x 8 q-tiles per XCD
    (2, 32, 1024, 128, A.FA_DTYPE_F16),
])
def test_table_at_two_qtiles_per_cu(lib, B, H, N, D, dtype):
    """Exactly two q-tiles per CU (64 per XCD on 32 CUs): the XCD placement
    table pairs each CU's q-tiles long with short; no CU runs alone."""
    pl = plan(lib, contiguous(B=B, H=H, N=N, D=D, dtype=dtype, causal=1))
    assert pl.xcd_heads == B * H // 8 and pl.n_items == 64
    check_table(pl, B, H, N, D, 1)
    lens = [pl.tile_end[i] - pl.tile_begin[i] for i in range(64)]
    assert all(lens[j] + lens[32 + j] == lens[0] + lens[32] for j in range(32))


@pytest.mark.parametrize("B,H,N,D,causal,dtype", [
    (1, 4, 2048, 128, 1, A.FA_DTYPE_F16),
    (1, 4, 4096, 128, 1, A.FA_DTYPE_BF16),
    (1, 4, 8192, 128, 1, A.FA_DTYPE_F16),    # 8-wave causal
    (1, 1, 16384, 64, 1, A.FA_DTYPE_F16),
    (1, 2, 4096, 128, 0, A.FA_DTYPE_F16),    # few heads, non-causal
    (1, 1, 16384, 128, 0, A.FA_DTYPE_BF16),  # many chunks per q-tile
    (2, 3, 3001, 64, 1, A.FA_DTYPE_BF16),    # ragged
    (1, 1, 32768, 128, 1, A.FA_DTYPE_F16),   # q-tiles beyond the item budget
])
def test_split_plans_are_complete(lib, B, H, N, D, causal, dtype):
    pl = plan(lib, contiguous(B=B, H=H, N=N, D=D, dtype=dtype, causal=causal))
    BM = pl.block_rows
    assert pl.xcd_heads == 0
    if (N + BM - 1) // BM >= A.FA_PLAN_MAX_ITEMS:
        assert pl.n_items == 0  # no item left for a second chunk: never split
        return
    check_plan(pl, B, H, N, D, causal)


@pytest.mark.parametrize("N", [1, 64, 127, 128, 129, 1000, 2047, 2048, 4095, 6000, 8191, 8192,
                               12000, 16384])
@pytest.mark.parametrize("causal", [0, 1])
@pytest.mark.parametrize("H", [1, 3, 16, 64])
def test_plan_sweep(lib, N, causal, H):
    """Whatever the shape, a plan is either empty or complete."""
    for D in (64, 128):
        for dtype in (A.FA_DTYPE_F16, A.FA_DTYPE_BF16):
            pl = plan(lib, contiguous(B=1, H=H, N=N, D=D, dtype=dtype, causal=causal))
            if pl.key_halves == 2:
                check_pair(pl, 1, H, N, causal)
            elif pl.xcd_heads:
                check_table(pl, 1, H, N, D, causal)
            elif pl.n_items:
                check_plan(pl, 1, H, N, D, causal)
            else:
                assert pl.workspace_bytes == 0 and pl.n_merge == 0 and pl.n_slots == 0


def test_more_cus_split_more(lib):
    """The split is a response to idle CUs: a machine with fewer CUs runs the
    same problem unsplit, a larger one splits it."""
    p = contiguous(B=1, H=4, N=3000, D=128, causal=1)
    assert plan(lib, p, cus=8).n_items == 0
    assert plan(lib, p, cus=256).n_items > 0
    big = plan(lib, p, cus=1024)
    check_plan(big, 1, 4, 3000, 128, 1)
    assert big.n_slots >= plan(lib, p, cus=256).n_slots


def test_plan_ignores_pointers_and_lse(lib):
    p1 = contiguous(B=1, H=8, N=3000, D=128, causal=1)
    p2 = contiguous(B=1, H=8, N=3000, D=128, causal=1, lse=False)
    p2.q = 0x7000000
    a, b = plan(lib, p1), plan(lib, p2)
    assert bytes(a) == bytes(b)


def test_plan_rejects(lib):
    out = A.FaFwdPlan()
    p = contiguous()
    assert lib.fa_fwd_plan(ctypes.byref(p), 256, None) == A.FA_ERR_NULL
    assert lib.fa_fwd_plan(ctypes.byref(p), 0, ctypes.byref(out)) == A.FA_ERR_ARG
    assert "compute_units" in lib.fa_last_error().decode()
    p.head_dim = 96
    assert lib.fa_fwd_plan(ctypes.byref(p), 256, ctypes.byref(out)) == A.FA_ERR_HEADDIM
    assert out.n_items == 0 and out.workspace_bytes == 0


def test_workspace_bound(lib):
    """Workspace per (batch, head) is at most kMaxSplitItems slots of BM rows:
    the plan never asks for more than B*H*128*256*(128*4+8) bytes."""
    for N in (2048, 3000, 4096, 8192, 16384):
        pl = plan(lib, contiguous(B=1, H=1, N=N, D=128, causal=0))
        assert pl.workspace_bytes <= 128 * 256 * (128 * 4 + 16)
        assert pl.n_slots <= A.FA_PLAN_MAX_ITEMS
