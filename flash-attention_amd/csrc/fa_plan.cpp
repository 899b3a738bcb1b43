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
  // The choice launch_causal makes.
  if (a.causal) return (!a.bf16 && a.seq_len >= kWideCausalMinSeq) ? 256 : 128;
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
      plan->merge_slot[n_merge] = (uint16_t)n_slots;
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
    plan->slot[i] = (uint16_t)(list[i].nch > 1 ? slot_base[list[i].qb] : 0);
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
//
// With allow_split the longest k q-tiles of every head may also be cut in
// two chunks, as long as the grid stays one round (n + k * heads_per_xcd
// <= 2 cpx); k is chosen by a model of the round: a workgroup alone costs
// 1 per key tile, two sharing a CU 1.85 each while both run (measured
// 1.14 us and 2.1 us per 128x64 tile), 1.5 per workgroup for its prologue,
// and a split adds the merge (about 3.5 tile times plus the partials'
// fp32 read-back at ~4 TB/s).  Returns the workspace bytes (0 unsplit).
size_t plan_xcd_table(const KernelArgs& a, int compute_units, bool allow_split,
                      SplitPlan* plan) {
  const int BM = block_rows(a);
  if (!a.causal || BM != 128 || compute_units % 8 != 0) return 0;
  const int64_t bh = (int64_t)a.batch * a.heads;
  if (bh % 8 != 0) return 0;
  const int nq = (a.seq_len + BM - 1) / BM;
  const int64_t hpx = bh / 8;
  const int64_t cpx = compute_units / 8;
  const int64_t n0 = hpx * nq;
  if (n0 <= cpx || n0 > 2 * cpx || n0 > kMaxSplitItems) return 0;
  const int k_max =
      allow_split ? (int)std::min<int64_t>(nq, (std::min<int64_t>(2 * cpx, kMaxSplitItems) - n0) / hpx)
                  : 0;
  constexpr double kShared = 2.1 / 1.14, kPrologue = 1.5, kMergeFixed = 3.5;
  const double tile_us = a.head_dim == 128 ? 1.14 : 0.62;
  struct Entry { int len, qb, head, c, nch; };
  Entry all[kMaxSplitItems];
  auto build = [&](int k) {  // the k longest q-tiles (the last k) of every head in two chunks
    int cnt = 0;
    for (int h = 0; h < (int)hpx; ++h)
      for (int qb = 0; qb < nq; ++qb) {
        const int T = q_tile_tiles(a, BM, qb);
        const int nch = qb >= nq - k ? 2 : 1;
        for (int c = 0; c < nch; ++c) {
          const int len = (int)((int64_t)(c + 1) * T / nch) - (int)((int64_t)c * T / nch);
          all[cnt++] = Entry{len, qb, h, c, nch};
        }
      }
    std::stable_sort(all, all + cnt, [](const Entry& x, const Entry& y) {
      return x.len != y.len ? x.len > y.len : (x.qb != y.qb ? x.qb > y.qb : x.c < y.c);
    });
    return cnt;
  };
  // Position of sorted entry src for n entries: alone positions take the
  // longest, then pairs longest-with-shortest.
  auto position_of = [&](int n, int src) {
    const int m = (int)(n - cpx) > 0 ? (int)(n - cpx) : 0;
    const int alone = (int)cpx - m;
    if (src < alone) return m + src;
    if (src < alone + m) return src - alone;
    return (int)cpx + (n - 1 - src);
  };
  auto model = [&](int k) {
    const int n = build(k);
    const int m = n > cpx ? n - (int)cpx : 0;
    const int alone = (int)cpx - m;
    double worst = 0.0;
    for (int i = 0; i < alone && i < n; ++i) worst = std::max(worst, all[i].len + kPrologue);
    for (int j = 0; j < m; ++j) {
      const double x = all[alone + j].len + kPrologue, y = all[n - 1 - j].len + kPrologue;
      worst = std::max(worst, std::min(x, y) * kShared + std::fabs(x - y));
    }
    if (k > 0) {
      const double bytes = (double)bh * 2 * k * BM * ((double)a.head_dim * 4 + 16);
      worst += kMergeFixed * 1.14 / tile_us + bytes / 4e12 / (tile_us * 1e-6);
    }
    return worst;
  };
  int best_k = 0;
  double best = model(0);
  for (int k = 1; k <= k_max; ++k) {
    const double c = model(k);
    if (c < best - 1e-9) {
      best = c;
      best_k = k;
    }
  }
  const int n = build(best_k);
  for (int src = 0; src < n; ++src) {
    const int pos = position_of(n, src);
    const Entry& e = all[src];
    plan->item[pos] = (uint32_t)e.qb | ((uint32_t)e.c << 16) | ((uint32_t)e.nch << 24);
    plan->slot[pos] = (uint16_t)e.head;
    // partial slots: 2 per split q-tile, in q-tile order (same for every head)
    plan->part[pos] = (uint16_t)(e.nch > 1 ? 2 * (e.qb - (nq - best_k)) : 0);
  }
  plan->n_items = n;
  plan->xcd_heads = (int)hpx;
  if (best_k == 0) return 0;
  for (int j = 0; j < best_k; ++j) {
    plan->merge[j] = (uint32_t)(nq - best_k + j) | (2u << 16);
    plan->merge_slot[j] = (uint16_t)(2 * j);
  }
  plan->n_merge = best_k;
  plan->n_slots = 2 * best_k;
  return (size_t)bh * plan->n_slots * BM * ((size_t)a.head_dim * 4 + 16);
}

}  // namespace

size_t plan_split(const KernelArgs& a, int compute_units, bool allow_split, SplitPlan* plan) {
  plan->n_items = plan->n_slots = plan->n_merge = plan->xcd_heads = 0;
  if (compute_units < 1) return 0;
  if (allow_split) {
    const size_t bytes = plan_chunks(a, compute_units, plan);
    if (bytes > 0) return bytes;
    plan->n_items = plan->n_slots = plan->n_merge = 0;
  }
  return plan_xcd_table(a, compute_units, allow_split, plan);
}

}  // namespace fa
