// Host-side work planning of the forward launches (no device code): the
// block height the launcher picks, the split-KV plan and the XCD placement
// table (declared in fa_fwd_kernel.h).  Pure host C++ so it can be built and
// checked on the CPU, including under AddressSanitizer.
//
// The reference launches one workgroup per q-tile
// (python/flash_attention_runtime/_ext.cu:96-102); these plans have no
// counterpart there.
#include <algorithm>
#include <cmath>
#include <cstdint>

#include "fa_fwd_kernel.h"

namespace fa {

int block_rows(const KernelArgs& a) {
  // The choice launch_causal makes.  Causal bf16 takes 8-wave workgroups on
  // long rows only where the 4-wave grid would be split: same box, against
  // 4 waves, B1 H2 N8192 +33 % (its split plan); but B1 H4 N8192 D64 (pair
  // mode) -4.9 %, B1 H8 N8192 (placement table) -2.9 %, B2 H32 N8192 (C4)
  // -0.7...0 %, and +1...+2 % for B2 H8 N8192 and B1 H16 N16384.
  if (a.causal) {
    if (a.seq_len < kWideCausalMinSeq) return 128;
    const int64_t tiles128 = (int64_t)a.batch * a.heads * ((a.seq_len + 127) / 128);
    return (!a.bf16 || tiles128 < kWideCausalBf16MaxTiles) ? 256 : 128;
  }
  return a.seq_len >= kWideMinSeq ? 256 : 128;
}

namespace {

constexpr int kKeyTile = 64;  // keys per K/V tile (Tile<D>::BN)

// Key tiles of q-tile qb.
int q_tile_tiles(const KernelArgs& a, int BM, int qb) {
  const int kv = a.causal ? std::min(a.seq_len, (qb + 1) * BM) : a.seq_len;
  return (kv + kKeyTile - 1) / kKeyTile;
}

// Split-KV plan, or 0 items when no split pays (see plan_split).
size_t plan_chunks(const KernelArgs& a, int compute_units, SplitPlan* plan) {
  const int BM = block_rows(a);
  const int nq = (a.seq_len + BM - 1) / BM;
  if (nq > kMaxSplitItems) return 0;
  auto tiles = [&](int qb) { return q_tile_tiles(a, BM, qb); };
  // Workgroup slots of the machine: two 4-wave workgroups or one 8-wave
  // workgroup per CU.  The unsplit grid finishes no earlier than its longest
  // q-tile (t_max key tiles) and no earlier than the total load over the
  // machine's throughput.  A CU running one 4-wave workgroup alone already
  // reaches ~90 % of its two-workgroup throughput (measured: 1.14 us per
  // 128x64 tile alone, 2.1 us each for two), so the throughput bound counts
  // 1.1 workgroups per CU for 4-wave kernels.  Split only when the longest
  // q-tile clearly dominates that bound: the partials cost an fp32 write
  // and read of O per chunk, which ate the whole gain at B1 H16 N3000
  // causal (bound ratio 1.4) and left +11 % at H8 (2.8) and +50 % at
  // B1 H4 N8192 causal (3.9).
  const int64_t slots = (int64_t)compute_units * (BM == 128 ? 2 : 1);
  int64_t sum = 0;
  int t_max = 0;
  for (int qb = 0; qb < nq; ++qb) {
    sum += tiles(qb);
    t_max = std::max(t_max, tiles(qb));
  }
  const double total = (double)sum * a.batch * a.heads;
  const double bound = total / ((double)compute_units * (BM == 128 ? 1.1 : 1.0));
  if (t_max <= 1.5 * bound + 8.0) return 0;
  const double avg = total / (double)slots;  // per workgroup slot
  // Chunks of at most S key tiles, S about the average load (at least 8
  // tiles, so the per-item prologue and the partial write stay small).
  int64_t S = std::max<int64_t>(8, (int64_t)std::ceil(avg));
  auto n_chunks = [&](int qb) { return (int)std::min<int64_t>(255, (tiles(qb) + S - 1) / S); };
  for (;;) {
    int64_t items = 0;
    for (int qb = 0; qb < nq; ++qb) items += n_chunks(qb);
    if (items <= kMaxSplitItems) break;
    S *= 2;
  }
  // Items, longest first (the dispatch order of the grid).
  struct Item { int len, qb, c, nch; };
  Item list[kMaxSplitItems];
  int n = 0, slot_base[kMaxSplitItems], n_slots = 0, n_merge = 0;
  for (int qb = 0; qb < nq; ++qb) {
    const int nch = n_chunks(qb), T = tiles(qb);
    slot_base[qb] = n_slots;
    if (nch > 1) {
      plan->merge[n_merge] = (uint32_t)qb | ((uint32_t)nch << 16);
      plan->merge_slot[n_merge] = (uint32_t)n_slots;
      ++n_merge;
      n_slots += nch;
    }
    for (int c = 0; c < nch; ++c) {
      // Same split of [0, T) as the kernel's t_begin / t_end.
      const int len = (int)((int64_t)(c + 1) * T / nch) - (int)((int64_t)c * T / nch);
      list[n++] = Item{len, qb, c, nch};
    }
  }
  if (n_merge == 0) return 0;
  std::stable_sort(list, list + n, [](const Item& x, const Item& y) {
    return x.len != y.len ? x.len > y.len : x.qb > y.qb;
  });
  for (int i = 0; i < n; ++i) {
    plan->item[i] = (uint32_t)list[i].qb | ((uint32_t)list[i].c << 16) |
                    ((uint32_t)list[i].nch << 24);
    plan->slot[i] = (uint32_t)(list[i].nch > 1 ? slot_base[list[i].qb] : 0);
  }
  plan->n_items = n;
  plan->n_slots = n_slots;
  plan->n_merge = n_merge;
  // Partial O (fp32) then (m, l, lr, unused) per row of every slot.
  return (size_t)a.batch * a.heads * n_slots * BM * ((size_t)a.head_dim * 4 + 16);
}

// XCD placement table for a causal 4-wave grid of one round: each XCD
// (cpx CUs) receives n = heads_per_xcd * nq workgroups, cpx < n <= 2 cpx.
// Measured dispatch (per-workgroup hardware CU ids): an XCD's k-th
// workgroup goes to CU slot k mod cpx, so positions k and k + cpx share a
// CU for k < n - cpx, and positions n - cpx .. cpx - 1 run alone.  Longest
// first (the default order) pairs the longest q-tile with the (cpx+1)-th
// longest: at B1 H16 N3000 the 47-tile q-tile shared its CU with a 32-tile
// one and set the kernel time (66 us).  The table gives the alone
// positions the longest items and pairs the rest longest with shortest.
// Grids of 0.75 to 2 q-tiles per CU run in pair mode (plan_split), so the
// table remains for n = 2 cpx, where no CU runs alone and the pairing is
// the whole gain.  No q-tile is split and the kernel's arithmetic is that
// of the plain grid (only the order changes).  Returns 0 (no workspace).
size_t plan_xcd_table(const KernelArgs& a, int compute_units, SplitPlan* plan) {
  const int BM = block_rows(a);
  if (!a.causal || BM != 128 || compute_units % 8 != 0) return 0;
  const int64_t bh = (int64_t)a.batch * a.heads;
  if (bh % 8 != 0) return 0;
  const int nq = (a.seq_len + BM - 1) / BM;
  const int64_t hpx = bh / 8;
  const int64_t cpx = compute_units / 8;
  const int64_t n = hpx * nq;
  if (n <= cpx || n > 2 * cpx || n > kMaxSplitItems) return 0;
  struct Entry { int len, qb, head; };
  Entry all[kMaxSplitItems];
  int cnt = 0;
  for (int h = 0; h < (int)hpx; ++h)
    for (int qb = 0; qb < nq; ++qb) all[cnt++] = Entry{q_tile_tiles(a, BM, qb), qb, h};
  std::stable_sort(all, all + cnt, [](const Entry& x, const Entry& y) {
    return x.len != y.len ? x.len > y.len : x.qb > y.qb;
  });
  // Sorted entry src goes to position: the alone positions take the
  // longest, then pairs longest-with-shortest.
  const int m = (int)(n - cpx);
  const int alone = (int)cpx - m;
  for (int src = 0; src < cnt; ++src) {
    const int pos = src < alone ? m + src : (src < alone + m ? src - alone : (int)cpx + (cnt - 1 - src));
    plan->item[pos] = (uint32_t)all[src].qb | (1u << 24);
    plan->slot[pos] = (uint32_t)all[src].head;
  }
  plan->n_items = cnt;
  plan->xcd_heads = (int)hpx;
  return 0;
}

}  // namespace

// Pair mode for causal 4-wave grids of 0.75 to 2 q-tiles (128 rows) per CU:
// one 8-wave workgroup per q-tile, its halves on alternate key tiles, one
// workgroup per CU, dispatched longest first.  Such grids are bound by
// their longest q-tiles, which a 4-wave workgroup runs alone on its CU
// once its partner is done (1.55 us per key tile alone against 2.1 us for
// each of two sharing it, at B1 H16 N3000); a pair workgroup keeps two waves
// on every SIMD.  Measured against the 4-wave kernel with its plans: +7..8 %
// at B1 H16 N3000 (Q, K ~ N(0, 3^2)), +8..27 % at H8..H16 N2048..6000
// (bf16 and D = 64 included); -6..-12 % at H24 and H32 N3000 (2.25 and 3 per
// CU) and -20..-49 % below 0.75 per CU (H4, H6), where split-KV spreads the
// few long q-tiles over more CUs.
namespace {
bool pair_mode(const KernelArgs& a, int compute_units) {
  if (!a.causal || block_rows(a) != 128) return false;
  const int64_t items = (int64_t)a.batch * a.heads * ((a.seq_len + 127) / 128);
  return 4 * items >= 3 * (int64_t)compute_units && items < 2 * (int64_t)compute_units;
}
}  // namespace

// Heads per dispatch group of an XCD for a causal grid in plain order (the
// kernel interleaves the q-tiles of a group's heads, longest first, and
// runs the groups one after the other).  Interleaving keeps a head's long
// q-tiles from starting late (+1.5 % at B2 H32 N8192 and B1 H16 N16384,
// +2.7 % at B1 H16 N8192 over head after head); smaller groups shrink the
// XCD's K/V working set.  Groups of 4 instead of all 8 heads of B2 H32
// N8192 measured +2.3…3 %, and groups of 2 another +0.4…1.3 % there (HBM
// reads 1.23 GB with groups of 4), but -1.5…1.8 % at B4 H32 N4096, where a
// group of 2 heads is a single round of workgroups: a group is kept at two
// or more rounds.
namespace {
int causal_head_group(const KernelArgs& a, int compute_units, bool pair) {
  const int64_t bh = (int64_t)a.batch * a.heads;
  if (!a.causal || bh % 8 != 0) return 0;
  const int hpx = (int)(bh / 8);  // heads per XCD
  int g = hpx % 4 == 0 ? 4 : hpx;
  const int bm = pair ? 128 : block_rows(a);
  const int64_t nq = (a.seq_len + bm - 1) / bm;
  const int64_t slots_per_xcd = (int64_t)(compute_units / 8) * (bm == 128 && !pair ? 2 : 1);
  if (g > 2 && hpx % 2 == 0 && 2 * nq >= 2 * slots_per_xcd) g = 2;
  return g;
}
}  // namespace

size_t plan_split(const KernelArgs& a, int compute_units, bool allow_split, SplitPlan* plan) {
  plan->n_items = plan->n_slots = plan->n_merge = plan->xcd_heads = plan->pair = 0;
  plan->head_group = 0;
  if (compute_units < 1) return 0;
  if (pair_mode(a, compute_units)) {
    plan->pair = 1;
    plan->head_group = causal_head_group(a, compute_units, true);
    return 0;
  }
  if (allow_split) {
    const size_t bytes = plan_chunks(a, compute_units, plan);
    if (bytes > 0) return bytes;
    plan->n_items = plan->n_slots = plan->n_merge = 0;
  }
  const size_t bytes = plan_xcd_table(a, compute_units, plan);
  if (plan->n_items == 0) plan->head_group = causal_head_group(a, compute_units, false);
  return bytes;
}

}  // namespace fa
