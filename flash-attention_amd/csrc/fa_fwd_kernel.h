// Internal interface between the C ABI (fa_api.cpp) and the HIP kernels.
// Mirrors the reference's kernel argument block ForwardKernelArgs
// (src/config/config.cuh:20-45) with 64-bit strides, dtype, LSE, the
// precomputed exponent scale and the split-KV work plan.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace fa {

// Work plan of a launch, computed on the host (plan_split).
//
// Split-KV: long key ranges of a q-tile are cut into chunks computed by
// separate workgroups, whose partial results (fp32 O normalised by the
// chunk's own row sum, offset m and row sum l per row) go to a
// caller-provided workspace and are merged by a second kernel.  Used when the grid would leave most of the machine idle
// behind a few long q-tiles (short causal problems, few heads).
//
// XCD placement table (xcd_heads > 0): a causal grid of exactly two q-tiles
// per CU, where the hardware puts the k-th and (k + CUs per XCD)-th
// workgroups of an XCD on the same CU.  The table orders each XCD's q-tiles
// so the longest run alone and the others share a CU long with short.
constexpr int kMaxSplitItems = 128;

struct SplitPlan {
  int32_t n_items;   // work items per (batch, head); 0: no split
  int32_t n_slots;   // partial-result slots per (batch, head)
  int32_t n_merge;   // q-tiles with more than one chunk (merged by the second kernel)
  int32_t xcd_heads; // > 0: XCD placement table over this many heads per XCD
  int32_t pair;      // 1: pair mode (8 waves per 128-row causal q-tile, no items)
  // Causal grids in plain order with B*H a multiple of 8 (no items, no
  // table): each XCD runs its heads in groups of head_group, the q-tiles of
  // a group's heads interleaved longest first; 0 otherwise.
  int32_t head_group;
  // Item i: q-tile (bits 0..15), chunk (16..23), chunk count (24..31).
  uint32_t item[kMaxSplitItems];
  // Item i's first partial slot of its q-tile (items of one q-tile use
  // slot[i] + chunk); unused for single-chunk items.  In the XCD placement
  // table: the head (within the XCD's heads) of dispatch position i.
  // 32-bit like every array here: the kernels read these arrays with scalar
  // loads at a wave-uniform index, and the compiler may fold a 16-bit
  // element's byte offset (2i) into the base address of a neighbouring
  // 32-bit load; scalar loads ignore the base's low two bits, so at odd i
  // that load returned element i - 1 (item[i] of the XCD placement table
  // with one head per XCD: every odd q-tile unwritten).
  uint32_t slot[kMaxSplitItems];
  // Merge list: q-tile (bits 0..15) | chunk count (16..23), first slot in merge_slot.
  uint32_t merge[kMaxSplitItems];
  uint32_t merge_slot[kMaxSplitItems];
};

struct KernelArgs {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  float* lse;
  // element strides: batch, head, seq (head_dim stride is 1)
  int64_t q_stride_b, q_stride_h, q_stride_s;
  int64_t k_stride_b, k_stride_h, k_stride_s;
  int64_t v_stride_b, v_stride_h, v_stride_s;
  int64_t o_stride_b, o_stride_h, o_stride_s;
  int32_t batch, heads, seq_len, head_dim;
  int32_t causal;
  int32_t bf16;
  int32_t n_qblocks;  // filled by the launcher
  float scale;        // softmax scale (natural units, used for the LSE)
  float scale_log2;   // softmax scale * log2(e), used for exp2
  // Split-KV (filled by the launcher when a workspace is used).
  float* ws_o;        // [batch*heads][n_slots][BM][head_dim] fp32 partial O
  float* ws_ml;       // [batch*heads][n_slots][BM][4] fp32 (m, l, lr, unused)
  SplitPlan split;
};

// Non-causal problems with at least this many keys use 8-wave workgroups;
// causal fp16 problems from kWideCausalMinSeq keys on, and causal bf16 ones
// from there when their grid of 128-row q-tiles has fewer than
// kWideCausalBf16MaxTiles of them (three per four CUs of an MI355X: such
// grids are split).
constexpr int kWideMinSeq = 2048;
constexpr int kWideCausalMinSeq = 8192;
constexpr int kWideCausalBf16MaxTiles = 192;

// Workgroup rows (BM) of the kernel variant launch_fwd picks for args.
int block_rows(const KernelArgs& args);

// Computes the work plan for args on a device with `compute_units` CUs
// (host code, fa_plan.cpp).
// Causal grids of 0.75 to 2 q-tiles per CU get pair mode (pair = 1, no
// items, returns 0) with or without a workspace.  Otherwise, with
// allow_split it may choose split-KV and returns the workspace bytes it
// needs; without (or when no split pays) it returns 0 and leaves either no
// plan (n_items = 0) or an XCD placement table (xcd_heads > 0).
size_t plan_split(const KernelArgs& args, int compute_units, bool allow_split, SplitPlan* plan);

// Launches the forward kernel for args (validated by the caller) on stream.
// With args.split.n_items > 0 (and the workspace set) it launches the split
// kernel and the merge kernel.
hipError_t launch_fwd(const KernelArgs& args, hipStream_t stream);

// Bytes of the library's static split-KV scratch array (per device).
constexpr size_t kScratchBytes = size_t(32) << 20;

// Device address of that array on the calling thread's current device
// (hipGetSymbolAddress on the first call per device, then cached).
hipError_t scratch_buffer(void** ptr);

}  // namespace fa
