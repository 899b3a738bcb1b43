// FlashAttention-2 forward for MI355X (gfx950 / CDNA4).
//
// Replaces the reference kernel flash_attention_forward_v6_mma
// (src/forward/forward_v6_mma.cuh:325-412) and its building blocks
// (src/loadstore, src/tensor_core, src/softmax, src/ptx).  It is written for
// the CDNA4 execution model rather than translated from the mma.sync design:
//
//  * One workgroup = NW wave64s, each wave owns 32 query rows (BM = 32*NW):
//    NW = 4 with two workgroups per CU, or NW = 8 (one workgroup per CU,
//    half the staging traffic per flop) for long rows (non-causal N >= 2048,
//    causal fp16 N >= 8192); either way two waves share each SIMD.
//  * S^T = K * Q^T on v_mfma_f32_32x32x16_{f16,bf16}: K tile rows are the A
//    operand (read from LDS), Q rows are the B operand (kept in VGPRs for the
//    whole kernel).  In the 32x32 accumulator layout lane l holds column
//    l%32 — one query row — and 16 keys, so the online-softmax row max and row
//    sum are in-lane; only lanes l and l^32 share a row (one cross-half swap).
//  * O^T += V^T * P^T on the same MFMA.  P^T is taken straight from the S^T
//    accumulator registers as the B operand: the MFMA contraction index is
//    mapped to keys by a fixed permutation sigma (k-slot 8g+t of lane group g
//    <-> key 8*(t/4) + 4g + t%4 inside each 16-key chunk), and the V^T A
//    operand is fetched with the same sigma using ds_read_b64_tr_b16, the
//    gfx950 transposing LDS read, so no register shuffle is needed.
//  * K and V tiles (64 keys) are staged by global_load_lds_dwordx4 (direct
//    global->LDS, 16 B per lane, no VGPR round trip) into a double-buffered
//    LDS ring; the loads of tile t+1 fly while tile t is computed.  Each tile
//    carries an XOR swizzle on its 16-byte chunks chosen so the K reads
//    (ds_read_b128) and the V transposed reads hit distinct banks.
//  * LDS operands are read a few MFMAs ahead of use (K: 3 k-steps, V: 4
//    MFMAs, the first V reads overlapping the softmax) so each MFMA finds its
//    operand ready, and wave priorities keep the two waves of a SIMD in
//    complementary phases (one wave's MFMAs while the other's softmax).
//  * Causal: fully-masked K tiles are never loaded or computed; q-tiles are
//    dispatched longest-first across each XCD's heads.  Ragged N: loads
//    clamp to the last row and the scores of keys >= N are -inf; rows >= N
//    are never stored.
//  * Block ids are remapped so each XCD (private L2) works on consecutive
//    q-tiles of the same heads.  Causal 4-wave grids of exactly two q-tiles
//    per CU follow an XCD placement table instead (q-tiles paired long with
//    short on each CU; see plan_xcd_table).
//  * Pair mode (causal grids of 0.75 to 2 q-tiles of 128 rows per CU): 8
//    waves run one q-tile, waves 0-3 on the even key tiles and waves 4-7 on
//    the odd ones, each half with its own K/V ring; the halves meet in LDS
//    at the end.  A long q-tile then never runs as a lone 4-wave workgroup
//    on its CU (one wave per SIMD), which set the time of such grids.
//  * O (and the fp32 split partials) leave through LDS: each wave parks its
//    32-row tile in the then idle K/V ring and stores whole rows, 16
//    contiguous bytes per lane.
//  * Split-KV (with a caller workspace, when a few long q-tiles would set
//    the time of a short grid): a q-tile's key tiles are cut into chunks
//    computed by separate workgroups, which write fp32 partials (O, m, l);
//    fa_merge_kernel combines them.
//
// Numerics follow the reference (src/softmax/online_softmax.cuh:13-19,
// :89-152; src/forward/forward_v6_mma.cuh:19-38): fp32 scores, an exponent
// offset m taken from the raw scores, p = exp2(s*c - m*c) with
// c = scale*log2(e), O and l rescaled by exp2((m_old - m_new)*c), P rounded
// to the input type with round-to-nearest-even before the PV product, O
// normalised in fp32 and rounded to the input type.  Differences: m is a
// lazy offset, raised only when a tile's P sums would reach kSumLimit (the
// common factor exp2(m_max*c - m*c) cancels in O/l), so the
// row max is computed only on such tiles (fp16 non-causal and fp16 causal in
// 8-wave workgroups run an optimistic pass with the offset of the first tile
// and redo the workgroup with per-tile checks only if a P overflowed); O is
// normalised by the sum of the rounded P (the weights P V actually uses: with
// the lazy offset the largest P of a row is not exactly 1, and this makes its
// rounding cancel); the LSE uses the sum of the unrounded p, as the
// reference's l, in the checked pass of bf16 and of fp16 at D = 64, and the
// rounded sum elsewhere (fp16, relative error <= 2^-11 per term); and the
// natural-log LSE = m*scale + ln(l) is new.

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>
#include <cmath>
#include <type_traits>

#include <atomic>
#include <mutex>

#include "fa_device_ops.h"
#include "fa_fwd_kernel.h"
#include "fa_lds_layout.h"

// Split-KV workspace of fa_fwd_scratch, for callers that cannot allocate:
// one array per GPU the library runs on, held until the process ends.  Host
// code never passes `scratch` itself (its host-side name is not a device
// address); it uses the address scratch_buffer() obtains per device.
static __device__ __align__(256) char scratch[fa::kScratchBytes];

namespace fa {
namespace {

using namespace dev;


using lds::Tile;
using lds::dma_slot;

// Lazy exponent offset.  The offset m in p = exp2(s*c - m*c) is re-derived
// from the row max only when a tile's P sum (per lane, 32 keys) reaches
// kSumLimit; every P then stays below it, finite in fp16 (max 65504) and
// far from overflow in the fp32 O and l accumulators.  When it is re-derived,
// m moves for every row whose max exceeds it (the rescale that follows is
// branch-free and multiplies every row anyway), to kHeadroom log2 units above
// that max in the checked pass: the largest p of the tile is then
// 2^-kHeadroom, and the scores can rise about 16 + kHeadroom units before the
// next re-derivation.  Measured same box, against moving m to the row max only for
// rows 8 units above it: B1 H16 N3000 causal with Q, K ~ N(0, 3^2) +4.3 % for
// the headroom and another +3.4 % for moving every row, causal B2 H16 N4096
// with those inputs +3.2 % and +6.4 %, B4 H32 N4096 with them +1.6 % and
// +2.0 %, C5 +0.7 % and +2.0 %, bf16 causal B2 H32 N8192 with them +0.9 % and
// +4.2 % (those gains with a headroom of 4).  The cost of the headroom is
// precision in the smallest p: fp16 p below 2^-14 are subnormal, so keys more
// than 14 - kHeadroom units under the row max keep fewer bits.  fp16 takes 1:
// rows with a few keys 10-30 units above a broad floor of thousands (an
// attention sink over a long context) measured 4.5x the emulated reference
// kernel's max-abs error and 6.4x its mean at 4, 2.2x at 2, and 1.0x at 1 and
// 0 (the bar is 2x); against 4, a headroom of 1 costs C5 1.0 %, C5r 1.9 %
// and 1.4...3.9 % on other Q, K ~ N(0, 3^2) problems (same box; N(0, 1)
// inputs unchanged).  bf16 p stay normal down to 2^-126 and keep 4.
// LDS-poison debug build (compiled with -DFA_LDS_POISON, shipped as
// libfa_mi355x_poison.so, never the product library): every wave fills the
// LDS bytes it is about to stage (K/V ring slots, staged Q, the output
// rows, the pair-mode combine area) with all-ones words, NaN in fp16, bf16
// and fp32, and waits for the fill before the staging write.  A read that
// raced ahead of its wait or barrier then sees NaN instead of the previous
// tile's plausible values; with correct synchronisation the output is bit
// for bit that of the product build.
#ifdef FA_LDS_POISON
constexpr bool kLdsPoison = true;
#else
constexpr bool kLdsPoison = false;
#endif

// 15 * 2^12: below fp16's largest finite value, 65504 (+1.3 % on B1 H16 N3000
// causal and +1.8 % on causal B2 H16 N4096 with Q, K ~ N(0, 3^2) over 2^15).
constexpr float kSumLimit = 61440.0f;
constexpr float kHeadroomF16 = 1.0f;
constexpr float kHeadroomBf16 = 4.0f;
template <bool BF16>
constexpr float kHeadroom = BF16 ? kHeadroomBf16 : kHeadroomF16;
static_assert(kSumLimit < 65504.0f, "a P below the sum limit must be finite in fp16");
static_assert(kHeadroomF16 >= 0.0f && kHeadroomF16 < 14.0f,
              "the largest P of a re-derived tile, 2^-kHeadroom, must stay a normal fp16");
static_assert(kHeadroomBf16 >= 0.0f && kHeadroomBf16 < 100.0f, "bf16 P must stay normal");

// The optimistic pass keeps the first key tile's row max as the offset for
// the whole row; it overflows when a later score exceeds that max by about
// 16/c.  The workgroup leaves it after its first tile (and recomputes that
// tile in the per-tile checked pass) when some row's first-tile scores
// spread widely: max minus mean above kOptSpreadLimit in log2 units.
// Gaussian scores of standard deviation sigma (in log2 units) give
// max - mean ~ 2.4 sigma over 64 keys and a later excess over the first max
// of ~2 sigma at N = 16384, so the limit keeps the optimistic pass up to
// sigma ~ 4 and sends the Q, K ~ N(0, 3^2) inputs of B1 H16 N16384
// (sigma ~ 13) to the checked pass after one tile instead of after a whole
// failed optimistic pass (measured 1.0 ms instead of 1.9 ms there).
constexpr float kOptSpreadLimit = 10.0f;

// Operand prefetch depths (measured best on MI355X): K operands for S^T are
// read 3 k-steps ahead, V^T operands 4 MFMAs ahead.
constexpr int kKWindow = 3;
constexpr int kVWindow = 4;


// SPLIT: the grid runs the work items of args.split (chunks of q-tiles);
// otherwise one workgroup per q-tile.  LSE_L (bf16 pair mode and split
// chunks, launches that write an LSE): the optimistic pass also keeps the
// sums of the unrounded p, which only the LSE uses.
template <int D, bool BF16, bool CAUSAL, int NW, bool SPLIT, bool PAIR = false, bool LSE_L = false>
__global__ void __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(2, 2)))
    fa_fwd_kernel(const KernelArgs args) {
  using T = Tile<D>;
  using Ops = ElemOps<BF16>;
  // PAIR: 8 waves on one 128-row q-tile; waves 0-3 take the even key tiles
  // of the item, waves 4-7 the odd ones, each half with its own K/V ring,
  // and the halves are combined through LDS at the end.
  static_assert(!PAIR || NW == 8, "pair mode runs 8 waves");
  constexpr int BM = PAIR ? 128 : 32 * NW;
  constexpr int NWD = PAIR ? 4 : NW;  // waves that stage one tile
  constexpr int BN = T::BN;
  constexpr int KSTEPS = D / 16;  // MFMA k-steps for S^T (k = head dim)
  constexpr int DBLK = D / 32;    // 32-wide head-dim blocks of O^T
  constexpr int ITERS = T::BYTES / (1024 * NWD);  // DMA instructions per wave per tile
  // Row sums of P in the per-tile checked pass.  O is always normalised by
  // the sum of the rounded P (the weights P V actually uses, so the weights
  // of a row sum to 1 and a dominant key's rounding cancels; with a lazy
  // offset the largest P of a row is not exactly 1 as in the reference).
  // bf16, and fp16 at D = 64, also keep fp32 sums of the unrounded p for the
  // tile check and the LSE, as the reference's l (online_softmax.cuh:135-152):
  // bf16's 8 significant bits would cost up to 2^-9 in the LSE, and at D = 64
  // the softmax is twice as dense per MFMA, where two v_add_f32 issue faster
  // than one v_dot2c_f32_f16 for the check (+8 % at B4 H16 N1024 D64).  fp16
  // at D = 128 uses the rounded sum (v_dot2c) for all three.
  constexpr bool kUnroundedSum = BF16 || D == 64;
  // fp16, 8-wave or non-causal: the row sums of the rounded P run on the
  // matrix core (row_sum_mfma, 4 small MFMAs per tile in place of 16 v_dot2c
  // or 32 v_add_f32; +3 % at B4 H32 N4096, +2.7 % at causal B1 H16 N16384,
  // +4 % at B4 H16 N1024 D64; neutral for the 4-wave causal kernel, which
  // keeps the checked pass), and the
  // kernel runs an optimistic pass first: the offset m is taken from the row
  // max of the first key tile only and never checked again.  The check
  // needs per-tile sums before the PV product, which the MFMA sums cannot
  // give in time; instead a P that overflowed fp16 makes its row's final
  // sum inf (or NaN), the workgroup votes, and if any row failed it recomputes
  // everything with the per-tile checked pass.  On inputs whose scores never
  // exceed the first tile's max by ~16/c in a row (e.g. the N(0, 1)
  // benchmark inputs) the second pass never runs.  fp16 pair mode keeps the
  // checked pass: on inputs that fail the spread test (B1 H16 N3000 with
  // Q, K ~ N(0, 3^2)) the optimistic pass and its restart cost 9 %, more
  // than it gains on N(0, 1) inputs (0..+8 %).
  // bf16 in pair mode and split chunks runs the optimistic pass too: bf16 P
  // share fp32's exponent range, so the first tile's offset overflows a P
  // only ~120 log2 units above that tile's max, where the accumulators turn
  // inf first; no spread test is needed, and the end-of-pass test also sums
  // |O| (O can overflow alone when |V| is large).  Same box, against the
  // checked pass, launches without an LSE (with one): pair mode B1 H16
  // N3000 +6 % (+1.4 %), with Q, K ~ N(0, 3^2) +12.5 % (+7.4 %), B1 H8
  // N4096 +6.8 %, B1 H4 N8192 D64 +11 %; split B1 H2 N8192 causal +6.2 %
  // (+0.9 %), B1 H1 N16384 causal +8.9 %, B1 H2 N4096 +1.8 % (+0.9 %).
  constexpr bool kMfmaSums = BF16 ? (PAIR || SPLIT) : (!CAUSAL || (NW == 8 && !PAIR));
  static_assert(!LSE_L || (BF16 && kMfmaSums), "LSE_L: bf16 kernels with an optimistic pass");
  // The first tile of a wave always re-derives the offset (it is -inf), so
  // P is computed only once there, after the row max.  Skipping the first
  // computation measured +0.5…3 % on 4-wave and pair-mode grids, -0.3…0.8 %
  // on the other 8-wave grids (a different register allocation of the loop),
  // where it stays off.  The output is bitwise the same either way.
  constexpr bool kSkipFirstExp = NW != 8 || PAIR;
  // Checked pass: keep p in fp32 past the check, so that a re-derivation
  // rescales it by alpha instead of computing 32 exp2 again.  Measured +2 %
  // on B1 H16 N16384 and +3…5 % on B1 H16 N3000 (causal, Q, K ~ N(0, 3^2)),
  // +6…10 % on narrower such grids.  The 32 extra live VGPRs fit the 8-wave
  // kernels (at most 254) and D = 64; the 4-wave D = 128 kernels would spill.
  constexpr bool kRescaleP = NW == 8 || D == 64;
  // bf16 checked pass on 4-wave D = 128 grids: the sum of the rounded P
  // (O's normaliser) is taken on the matrix core, 4 row_sum_mfma per tile, in
  // place of 16 v_dot2c; the check and the LSE keep the unrounded fp32 sum.
  // The sums are rescaled with O on a re-derivation.  Measured +0.7…1.1 % at
  // C4, up to +4.7 % with Q, K ~ N(0, 3^2); -1 % on split grids (few heads),
  // which keep v_dot2c.  The 8-wave and D = 64 kernels have no VGPRs left
  // for it next to kRescaleP.
  constexpr bool kMfmaNorm = kUnroundedSum && !kRescaleP && !SPLIT;
  static_assert(ITERS >= 1 && T::BYTES % (1024 * NWD) == 0, "tile must split evenly over waves");

  // LDS ring: K buffers 0/1 then V buffers 0/1 (pair mode: K 0/1 of each
  // half, then V 0/1 of each half).
  __shared__ __attribute__((aligned(1024))) char smem[(PAIR ? 8 : 4) * T::BYTES];
  // Set by any wave whose optimistic pass left a row with a non-finite sum.
  __shared__ int redo_flag;
  if (kMfmaSums && threadIdx.x == 0) redo_flag = 0;  // ordered by the first barrier

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // Wave priorities.  8-wave workgroups: waves 4..7 (the second wave of each
  // SIMD) run at raised priority throughout, so when both waves of a SIMD
  // have MFMAs ready one of them streams ahead and the two drift into
  // complementary phases (+0.6..1 % over the per-phase scheme at
  // B4 H32 N4096).  4-wave workgroups, whose SIMD partner belongs to another
  // workgroup, raise the priority only while issuing PV MFMAs (below).
  if (NW == 8 && wave >= 4) __builtin_amdgcn_s_setprio(1);
  const int half = PAIR ? (wave >> 2) : 0;  // key-tile half (pair mode)
  const int rw = PAIR ? (wave & 3) : wave;   // 32-row block of the q-tile
  const int kslot = PAIR ? 2 * half : 0;     // this half's K ring slots
  const int vslot = PAIR ? 4 + 2 * half : 2;  // and V ring slots
  const int l32 = lane & 31;
  const int g = lane >> 5;         // which half of the wave
  const int lj = lane & 15;        // lane within its 16-lane group
  const int hg = (lane >> 4) & 1;  // 16-lane group within the half

  const int N = args.seq_len;
  // Work item of this workgroup: a q-tile, or with a plan one entry of its
  // table: a chunk of a q-tile's key tiles (split-KV; the plan lists items
  // longest first), or the q-tile of this dispatch position within its XCD
  // (XCD placement table).
  int bh, item;
  if (SPLIT && args.split.xcd_heads > 0) {
    // Hardware dispatch: workgroup b runs on XCD b % 8 as its (b / 8)-th.
    item = (int)(blockIdx.x >> 3);
    bh = (int)(blockIdx.x & 7) * args.split.xcd_heads + args.split.slot[item];
  } else {
    const int logical = xcd_remap(blockIdx.x, gridDim.x);
    const int per_bh = SPLIT ? args.split.n_items : args.n_qblocks;
    bh = logical / per_bh;
    item = logical - bh * per_bh;
  }
  int qb, chunk = 0, n_chunks = 1;
  if constexpr (SPLIT) {
    const uint32_t info = args.split.item[item];
    qb = (int)(info & 0xffffu);
    chunk = (int)((info >> 16) & 0xffu);
    n_chunks = (int)(info >> 24);
  } else {
    qb = CAUSAL ? args.n_qblocks - 1 - item : item;  // longest q-tiles first
    if (CAUSAL && ((args.batch * args.heads) & 7) == 0) {
      // Whole heads per XCD, taken in groups of args.split.head_group (the
      // plan's choice; all of them if it does not divide their count):
      // longest first across a group's heads (their q-tiles interleaved),
      // group after group.  Same blocks per XCD as xcd_remap.
      const int hpx = (args.batch * args.heads) >> 3;
      const int hg = args.split.head_group;
      const int grp_heads = hg > 0 && hpx % hg == 0 ? hg : hpx;
      const int per_grp = grp_heads * args.n_qblocks;
      const int i = (int)(blockIdx.x >> 3);
      const int grp = i / per_grp, w = i - grp * per_grp;
      bh = (int)(blockIdx.x & 7) * hpx + grp * grp_heads + w % grp_heads;
      qb = args.n_qblocks - 1 - w / grp_heads;
    }
  }
  const int b = bh / args.heads;
  const int h = bh - b * args.heads;

  const char* __restrict__ qh = reinterpret_cast<const char*>(args.q) +
                                2 * (b * args.q_stride_b + h * args.q_stride_h);
  const char* __restrict__ kh = reinterpret_cast<const char*>(args.k) +
                                2 * (b * args.k_stride_b + h * args.k_stride_h);
  const char* __restrict__ vh = reinterpret_cast<const char*>(args.v) +
                                2 * (b * args.v_stride_b + h * args.v_stride_h);
  char* __restrict__ oh = reinterpret_cast<char*>(args.o) +
                          2 * (b * args.o_stride_b + h * args.o_stride_h);
  const int64_t qsb = 2 * args.q_stride_s, ksb = 2 * args.k_stride_s;
  const int64_t vsb = 2 * args.v_stride_s, osb = 2 * args.o_stride_s;

  const int q0 = qb * BM;
  const int wrow0 = q0 + rw * 32;  // first query row of this wave
  const int qrow = wrow0 + l32;      // this lane's query row
  const int kv_end = CAUSAL ? min(N, q0 + BM) : N;
  const int q_tiles = (kv_end + BN - 1) / BN;  // key tiles of this q-tile
  // This item's key tiles [t_begin, t_end): chunk of n_chunks near-equal parts.
  const int t_begin = (int)((int64_t)chunk * q_tiles / n_chunks);
  const int t_end = (int)((int64_t)(chunk + 1) * q_tiles / n_chunks);
  // This wave's tiles: t_first, t_first + TS, ... (pair mode: every other
  // one), in n_steps steps shared by all waves of the workgroup.
  constexpr int TS = PAIR ? 2 : 1;
  const int t_first = t_begin + half;
  const int n_steps = PAIR ? (t_end - t_begin + 1) / 2 : t_end - t_begin;

  // ---- DMA plan: per-lane 32-bit source offsets within a tile ----
  uint32_t k_src[ITERS], v_src[ITERS];
#pragma unroll
  for (int it = 0; it < ITERS; ++it) {
    int r, c;
    dma_slot<D, NWD, false>(rw, it, lane, r, c);
    k_src[it] = (uint32_t)(r * ksb + c * 16);
    dma_slot<D, NWD, true>(rw, it, lane, r, c);
    v_src[it] = (uint32_t)(r * vsb + c * 16);
  }
  const uint32_t smem_base = __builtin_amdgcn_readfirstlane(lds_addr(smem));
  const uint32_t wave_dma_base = smem_base + rw * ITERS * 1024;
  // kLdsPoison: fill the KiB at LDS byte offset `off` (from smem), 16 bytes
  // per lane, as one wave's staging instruction covers it.
  auto poison_kib = [&](uint32_t off) FA_INLINE {
    *reinterpret_cast<u32x4*>(smem + off + lane * 16) = u32x4{~0u, ~0u, ~0u, ~0u};
  };

  // Stage K and V rows [t*BN, t*BN + BN) into LDS buffer `buf`.
  auto issue_tile = [&](int t, int buf) FA_INLINE {
    const int row0 = t * BN;
    const char* kbase = kh + row0 * ksb;
    const char* vbase = vh + row0 * vsb;
    const uint32_t kdst = wave_dma_base + (kslot + buf) * T::BYTES;
    const uint32_t vdst = wave_dma_base + (vslot + buf) * T::BYTES;
    if constexpr (kLdsPoison) {
#pragma unroll
      for (int it = 0; it < ITERS; ++it) {
        poison_kib(kdst - smem_base + it * 1024);
        poison_kib(vdst - smem_base + it * 1024);
      }
      __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the fill lands before the DMA
    }
    if (row0 + BN <= N) {
#pragma unroll
      for (int it = 0; it < ITERS; ++it) dma_16b(k_src[it], kbase, kdst + it * 1024);
#pragma unroll
      for (int it = 0; it < ITERS; ++it) dma_16b(v_src[it], vbase, vdst + it * 1024);
    } else {
      // ragged tail: rows past N re-read row N-1 (their scores are masked).
      // This lane's tile row for instruction it is it*RPI + r_lane.
      constexpr int RPI = 1024 / T::ROWB;  // rows per DMA instruction
      const int r_lane = (rw * ITERS) * RPI + lane / (T::ROWB / 16);
      const int last = N - 1 - row0;
#pragma unroll
      for (int it = 0; it < ITERS; ++it) {
        const int over = max(it * RPI + r_lane - last, 0);
        dma_16b(k_src[it] - (uint32_t)(over * ksb), kbase, kdst + it * 1024);
        dma_16b(v_src[it] - (uint32_t)(over * vsb), vbase, vdst + it * 1024);
      }
    }
  };

  // Start streaming the first tile while Q is fetched into registers.
  if (!PAIR || t_first < t_end) issue_tile(t_first, 0);

  // Q as the B operand of S^T = K Q^T: lane holds query qrow, dims
  // [16*kk + 8*g, +8) for k-step kk.  Read straight from global memory
  // that is 32 rows x 32 bytes per instruction.  4-wave workgroups instead
  // stage each wave's 32 rows in LDS with whole-row DMA (16 bytes per lane,
  // QRB / 16 lanes per row) and read the operands from there once they have
  // landed (+1.5..2.5 % at B4 H16 N1024 D64 and B1 H16 N3000 causal; the
  // 8-wave kernel, whose prologue is a small part of a long workgroup, loses
  // 0.5 % to it and keeps the direct loads).  The staging area, ring
  // buffers 1 and 3, is free until the first tile_step.  The rows form an
  // lds::row_tile_offset tile, so the operand reads (32 rows, one chunk
  // each) are conflict free.  Rows past N re-read row N-1.
  constexpr bool kStageQ = NW == 4;
  constexpr int QRB = 2 * D;  // bytes per Q row
  const uint32_t q_lds = (uint32_t)((wave < 2 ? 1 : 3) * T::BYTES + (wave & 1) * 32 * QRB);
  if constexpr (kStageQ) {
    const int qr0 = min(wrow0, N - 1);
    const char* qbase = qh + qr0 * qsb;
    if constexpr (kLdsPoison) {
#pragma unroll
      for (int it = 0; it < KSTEPS; ++it) poison_kib(q_lds + it * 1024);
      __builtin_amdgcn_s_waitcnt(0xc07f);
    }
#pragma unroll
    for (int it = 0; it < KSTEPS; ++it) {  // 32 rows x QRB bytes = KSTEPS x 1 KiB
      // DMA lane destinations are fixed (16 bytes per lane): fetch the chunk
      // that belongs at this position.
      const int pos = it * 1024 + lane * 16;
      const int r = pos / QRB, cs = (pos % QRB) / 16;
      const int row = min(wrow0 + r, N - 1) - qr0;
      dma_16b((uint32_t)(row * qsb + (cs ^ lds::row_swz(r, QRB)) * 16), qbase,
              smem_base + q_lds + it * 1024);
    }
  }
  i16x8 qf[KSTEPS];
  if constexpr (!kStageQ) {
    const int qr = qrow < N ? qrow : N - 1;
    const char* qp = qh + qr * qsb + g * 16;
#pragma unroll
    for (int kk = 0; kk < KSTEPS; ++kk)
      qf[kk] = *reinterpret_cast<const i16x8*>(qp + kk * 32);
  }

  f32x16 o_acc[DBLK];
#pragma unroll
  for (int db = 0; db < DBLK; ++db)
#pragma unroll
    for (int i = 0; i < 16; ++i) o_acc[db][i] = 0.0f;
  const float c = args.scale_log2;
  float m_run = -INFINITY;  // offset used in the exponent (<= the running max)
  float neg_mc = INFINITY;  // -m_run * c; +inf while m_run = -inf (trips the first check)
  float l_run = 0.0f;       // this lane's partial sum of P (unrounded p when kUnroundedSum)
  float lr_run = 0.0f;      // kUnroundedSum: this lane's partial sum of the rounded P
  f32x4 l_mfma = {0.0f, 0.0f, 0.0f, 0.0f};  // row sums on the matrix core (kMfmaSums, kMfmaNorm)
  const i16x8 sum_sel = row_sum_selector<BF16>(lane);

  // Per-lane LDS byte offsets inside a tile (loop invariant).
  // K: A operand of key block 0, k-step kk (block 1: + 32 rows).
  int k_off[KSTEPS];
#pragma unroll
  for (int kk = 0; kk < KSTEPS; ++kk) k_off[kk] = lds::k_read_offset<D>(0, kk, lane);
  // V^T: transposed read of chunk 0, half 0, head-dim block db (other chunks
  // and halves: + 16ch + 8hf rows, as immediates).
  uint32_t v_addr[DBLK];
#pragma unroll
  for (int db = 0; db < DBLK; ++db)
    v_addr[db] = smem_base + lds::v_read_offset<D>(0, 0, db, lane) + (vslot - 2) * T::BYTES;

  if constexpr (kStageQ) {
    // This wave's Q rows have landed (its own DMA): read the operands, and
    // finish the reads before the barrier after which tile 1 refills
    // buffers 1 and 3.
    __builtin_amdgcn_s_waitcnt(0);
#pragma unroll
    for (int kk = 0; kk < KSTEPS; ++kk)
      qf[kk] = *reinterpret_cast<const i16x8*>(smem + q_lds +
                                               lds::row_tile_offset(l32, 2 * kk + g, QRB));
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  // OPT: the optimistic pass of kMfmaSums kernels (offset from the first
  // tile only, row sums on the matrix core); otherwise every tile checks its
  // P sums before the PV product.
  auto compute_tile = [&](auto buf_c, int t, auto opt_c) FA_INLINE {
    constexpr int BUF = decltype(buf_c)::value;
    constexpr bool OPT = decltype(opt_c)::value;
    static_assert(!OPT || kMfmaSums, "the optimistic pass needs the matrix-core sums");
    const int kt0 = t * BN;
    const char* kt = smem + (kslot + BUF) * T::BYTES;

    // ---- S^T = K Q^T : two 32-key blocks ----
    // The K operands are read kKWindow k-steps ahead of their MFMA; the
    // sched_barriers keep the compiler from sinking each LDS read next to
    // its use (which would expose the full LDS latency on every MFMA).
    f32x16 s[2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int i = 0; i < 16; ++i) s[kb][i] = 0.0f;
    {
      constexpr int KD = kKWindow;
      i16x8 ka[KD][2];
      static_for<0, KD>([&](auto i_c) {
        constexpr int i = decltype(i_c)::value;
        if constexpr (i < KSTEPS) {
          ka[i][0] = *reinterpret_cast<const i16x8*>(kt + k_off[i]);
          ka[i][1] = *reinterpret_cast<const i16x8*>(kt + 32 * T::ROWB + k_off[i]);
        }
      });
      __builtin_amdgcn_sched_barrier(0);
      static_for<0, KSTEPS>([&](auto kk_c) {
        constexpr int kk = decltype(kk_c)::value;
        s[0] = Ops::mfma(ka[kk % KD][0], qf[kk], s[0]);
        s[1] = Ops::mfma(ka[kk % KD][1], qf[kk], s[1]);
        if constexpr (kk + KD < KSTEPS) {
          ka[kk % KD][0] = *reinterpret_cast<const i16x8*>(kt + k_off[kk + KD]);
          ka[kk % KD][1] = *reinterpret_cast<const i16x8*>(kt + 32 * T::ROWB + k_off[kk + KD]);
        }
        __builtin_amdgcn_sched_barrier(0);
      });
    }
    // Prefetch the first kVWindow V^T operands: their LDS latency hides
    // behind the softmax.
    constexpr int VD = kVWindow;
    constexpr int NPV = DBLK * 4;
    i16x8 va[VD];
    static_for<0, VD>([&](auto i_c) {
      constexpr int i = decltype(i_c)::value;
      constexpr int db = i % DBLK, ch = i / DBLK;
      constexpr int off = (2 + BUF) * T::BYTES + ch * 16 * T::ROWB;
      va[i] = ds_read_tr_pair<off, off + 8 * T::ROWB>(v_addr[db]);
    });
    __builtin_amdgcn_sched_barrier(0);

    // ---- masking (ragged tail / causal diagonal) ----
    const bool need_mask = (kt0 + BN > N) || (CAUSAL && kt0 + BN - 1 > wrow0);
    if (need_mask) {
      // Score (kb, i) holds key kt0 + 4g + off with the compile-time offset
      // off = 32kb + 8(i >> 2) + (i & 3); it is masked when the key exceeds
      // N - 1 or (causal) the row.  One per-lane limit then leaves a compare
      // and a select per score.
      const int last = (CAUSAL ? min(N - 1, qrow) : N - 1) - kt0 - 4 * g;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int off = kb * 32 + 8 * (i >> 2) + (i & 3);
          if (off > last) s[kb][i] = -INFINITY;
        }
    }

    // ---- P = exp2(s*c - m*c) with the current offset m, and its tile sums ----
    // P is packed as the P^T B operand: chunk ch = 2kb + hh uses S registers
    // 8hh..8hh+7 of block kb.  t0/t1 sum this lane's even/odd keys.
    // pack(pval) packs the fp32 p given by pval(kb, i) and, in the checked
    // pass, sums them.
    i16x8 pf[4];
    float t0, t1, tr;
    auto pack = [&](auto pval) FA_INLINE {
      t0 = 0.0f;
      t1 = 0.0f;
      tr = 0.0f;
#pragma unroll
      for (int ch = 0; ch < 4; ++ch) {
        const int kb = ch >> 1, base = (ch & 1) * 8;
        u32x4 w;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const float p0 = pval(kb, base + 2 * j);
          const float p1 = pval(kb, base + 2 * j + 1);
          w[j] = pack2<BF16>(p0, p1);
          if constexpr (kUnroundedSum && (!OPT || LSE_L)) {
            // Sum the unrounded fp32 p, as the reference does
            // (online_softmax.cuh:135-152), for the check and the LSE, and
            // the rounded P for the normalisation (optimistic pass: the LSE
            // only; the matrix core sums the rounded P).
            t0 += p0;
            t1 += p1;
            if constexpr (!kMfmaNorm && !OPT) tr = dot2_acc<BF16>(w[j], tr);
          }
        }
        pf[ch] = __builtin_bit_cast(i16x8, w);
        if constexpr (!kUnroundedSum && !OPT) {
          // fp16, D = 128: sum the rounded P (the values that enter P V;
          // relative error <= 2^-11 per term) with v_dot2c_f32_f16.
          t0 = dot2_acc<BF16>(w[0], t0);
          t1 = dot2_acc<BF16>(w[1], t1);
          t0 = dot2_acc<BF16>(w[2], t0);
          t1 = dot2_acc<BF16>(w[3], t1);
        }
      }
    };
    // p computed as it is packed (no fp32 copy kept).
    auto exp_pack = [&](float nmc) FA_INLINE {
      pack([&](int kb, int i) FA_INLINE { return fast_exp2(fmaf(s[kb][i], c, nmc)); });
    };
    // kRescaleP: p in fp32 (pv), kept past the check, packed by pack_pv.
    float pv[2][16];
    auto exp_f32 = [&](float nmc) FA_INLINE {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int i = 0; i < 16; ++i) pv[kb][i] = fast_exp2(fmaf(s[kb][i], c, nmc));
    };
    auto pack_pv = [&]() FA_INLINE { pack([&](int kb, int i) FA_INLINE { return pv[kb][i]; }); };

    // ---- online softmax with a lazy offset (reference online_softmax.cuh:89-152) ----
    // m need not be the running max: any m <= it gives the same O and l up
    // to a common factor that cancels in O / l.  It only has to keep every P
    // finite and below kSumLimit.  The tile sums check exactly that (a sum
    // bounds each of its terms, and is inf or NaN if a P overflowed or
    // m = -inf), so the row max is taken only when a sum reaches the limit:
    // on the first tile of a row, or when the scores jump by more than
    // ~(16 + kHeadroom)/c.  Then m moves (to kHeadroom above the row max in
    // the checked pass) for every row whose max exceeds it, O and l are
    // rescaled, and P is recomputed (kRescaleP: rescaled).
    bool rederive = true;
    if (!kSkipFirstExp || t != t_first) {
      if constexpr (OPT) {
        exp_pack(neg_mc);
        rederive = t == t_first;  // the first tile of every wave that computes any
      } else if constexpr (!kRescaleP) {
        exp_pack(neg_mc);
        rederive = __any(!(t0 + t1 < kSumLimit));
      } else {
        exp_f32(neg_mc);
        pack_pv();
        rederive = __any(!(t0 + t1 < kSumLimit));
      }
    }
    if (rederive) {
      // (In the optimistic pass this is the first tile: O and the sums are
      // still 0, so the rescale below is a no-op for them.)
      const float mx = pair_max(max32(s[0], s[1]));
      if constexpr (OPT && !BF16) {
        // Spread test (kOptSpreadLimit) on the first tile, with the mean
        // estimated from 8 of the row's 64 keys (keys 4g, 4g+9, 4g+50,
        // 4g+59 of each lane half): a wave that fails it asks the workgroup
        // to leave the optimistic pass after this tile.  -inf (masked)
        // scores make the mean -inf and fail it.
        const float sm = (s[0][0] + s[0][5]) + (s[1][10] + s[1][15]);
        const float mean = pair_sum(sm) * (1.0f / 8.0f);
        if (__any(!((mx - mean) * c <= kOptSpreadLimit)) && lane == 0) redo_flag = 1;
      }
      const float m_old = m_run;
      const bool grow = mx > m_run;  // false when both are -inf
      const float m_new = grow ? (OPT ? mx : mx + kHeadroom<BF16> / c) : m_run;
      // exp2(0) = 1 for rows that keep their offset (branch-free: also
      // covers m_run = -inf, where m_run - m_new would be NaN).
      const float alpha = fast_exp2(grow ? (m_run - m_new) * c : 0.0f);
      m_run = m_new;
      l_run *= alpha;
      if constexpr (kUnroundedSum && !kMfmaNorm) lr_run *= alpha;
      if constexpr (kMfmaNorm && !OPT) l_mfma = row_sum_scale(l_mfma, alpha, lane);
#pragma unroll
      for (int db = 0; db < DBLK; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) o_acc[db][i] *= alpha;
      // A row whose keys were all masked keeps m = -inf: its P is 0 now
      // (offset 0) and its next tile trips the check again (offset +inf).
      const bool none = m_run == -INFINITY;
      neg_mc = none ? INFINITY : -m_run * c;
      if constexpr (OPT || !kRescaleP) {
        exp_pack(none ? 0.0f : neg_mc);
      } else {
        // While the offset moves by less than 126 log2 units, p with the old
        // offset is finite (and within fp32 rounding of the exact value) and
        // alpha (<= 1) is a normal float, so the new p is the old one times
        // alpha.  Otherwise (the first tile, m_old = -inf, or a jump of the
        // scores) p is computed again from the scores: v_exp_f32 flushes a
        // result below 2^-126 to 0, and the offset sits kHeadroom above the
        // row max, so testing the max's jump alone would let a jump within
        // kHeadroom below 126 units zero the tile that holds the row's new
        // max.
        const bool recompute = !((m_new - m_old) * c < 126.0f);
        if ((kSkipFirstExp && t == t_first) || __any(recompute)) {
          exp_f32(none ? 0.0f : neg_mc);
        } else {
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int i = 0; i < 16; ++i) pv[kb][i] *= alpha;
        }
        pack_pv();
      }
    }
    if constexpr (!OPT || LSE_L) l_run += t0 + t1;
    if constexpr (!OPT && kUnroundedSum && !kMfmaNorm) lr_run += tr;

    // ---- O^T += V^T P^T ----
    // 4-wave workgroups: raised wave priority while this wave issues its PV
    // MFMAs: the other wave on the SIMD is then usually in its softmax
    // (VALU), and the arbiter keeps the matrix pipe fed from this one.
    if constexpr (NW != 8) __builtin_amdgcn_s_setprio(1);
    __builtin_amdgcn_sched_barrier(0);
    static_for<0, NPV>([&](auto j_c) {
      constexpr int j = decltype(j_c)::value;
      constexpr int db = j % DBLK, ch = j / DBLK;
      o_acc[db] = Ops::mfma(va[j % VD], pf[ch], o_acc[db]);
      if constexpr ((OPT || kMfmaNorm) && db == DBLK - 1)
        l_mfma = row_sum_mfma<BF16>(sum_sel, pf[ch], l_mfma);
      if constexpr (j + VD < NPV) {
        constexpr int db2 = (j + VD) % DBLK, ch2 = (j + VD) / DBLK;
        constexpr int off = (2 + BUF) * T::BYTES + ch2 * 16 * T::ROWB;
        va[j % VD] = ds_read_tr_pair<off, off + 8 * T::ROWB>(v_addr[db2]);
      }
      __builtin_amdgcn_sched_barrier(0);
    });
    if constexpr (NW != 8) __builtin_amdgcn_s_setprio(0);
  };

  auto tile_step = [&](auto buf_c, int t, auto opt_c) FA_INLINE {
    constexpr int BUF = decltype(buf_c)::value;
    if (t + TS < t_end) issue_tile(t + TS, BUF ^ 1);
    // Skip tiles whose every key lies after every row of this wave.
    if ((!PAIR || t < t_end) && (!CAUSAL || t * BN <= wrow0 + 31)) compute_tile(buf_c, t, opt_c);
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
  };
  auto run_tiles = [&](auto opt_c) FA_INLINE {
    constexpr bool OPT = decltype(opt_c)::value;
    for (int u = 0; u < n_steps; u += 2) {
      const int t = t_first + TS * u;
      tile_step(std::integral_constant<int, 0>{}, t, opt_c);
      // Optimistic pass: leave it after the first tile if a wave's spread
      // test failed (the flag was set before the tile's closing barrier).
      if constexpr (OPT)
        if (u == 0 && __builtin_amdgcn_readfirstlane(redo_flag) != 0) break;
      if (u + 1 < n_steps) tile_step(std::integral_constant<int, 1>{}, t + TS, opt_c);
    }
  };
  // l_tot: the row sum for the LSE; lr_tot: the sum of the rounded P, which
  // normalises O (the same value unless kUnroundedSum).
  float l_tot, lr_tot;
  if constexpr (kMfmaSums) {
    run_tiles(std::true_type{});
    l_tot = row_sum_of_lane(l_mfma, lane);
    // Vote: did any row of the workgroup overflow (or did the spread test
    // end the pass early)?  The loop ended with a barrier, so every wave is
    // done with the K/V ring.  bf16: also a sum of |O| that is not finite,
    // and (LSE_L) the LSE's sum of the unrounded p.
    bool bad = !(l_tot < INFINITY);
    if constexpr (BF16) {
      float sa = 0.0f;
#pragma unroll
      for (int db = 0; db < DBLK; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) sa += fabsf(o_acc[db][i]);
      bad = bad || !(sa < INFINITY);
    }
    lr_tot = l_tot;
    if constexpr (LSE_L) {
      l_tot = pair_sum(l_run);
      bad = bad || !(l_tot < INFINITY);
    }
    if (__any(bad) && lane == 0) redo_flag = 1;
    __syncthreads();
    if (redo_flag != 0) {
#pragma unroll
      for (int db = 0; db < DBLK; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) o_acc[db][i] = 0.0f;
      l_mfma = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      m_run = -INFINITY;
      neg_mc = INFINITY;
      l_run = 0.0f;
      lr_run = 0.0f;
      if (!PAIR || t_first < t_end) issue_tile(t_first, 0);
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      run_tiles(std::false_type{});
      l_tot = pair_sum(l_run);
      lr_tot = kUnroundedSum ? pair_sum(lr_run) : l_tot;
    }
  } else {
    run_tiles(std::false_type{});
    l_tot = pair_sum(l_run);
    lr_tot = kMfmaNorm ? row_sum_of_lane(l_mfma, lane) : kUnroundedSum ? pair_sum(lr_run) : l_tot;
  }

  // A partial result (a pair half, a split chunk) normalised by its own sum
  // of the rounded P, that sum's log moved into the offset: m' = m +
  // log2(lr) / c, O / lr, l / lr, lr' = 1 (m' = -inf, l = 0 where no key was
  // visible).  Combining partials weights each by exp2((m' - m'_max) c),
  // which leaves fp32's normal range (v_exp_f32 returns 0 below 2^-126)
  // only for a partial whose share of the row is that small.  Unnormalised,
  // bf16's optimistic pass (sums up to 2^127 at the offset of its first
  // tile, which can lie far below the row max) could lose a partial that
  // held a significant share.
  float part_inv = 0.0f;
  auto normalise_part = [&]() FA_INLINE {
    part_inv = lr_tot > 0.0f ? 1.0f / lr_tot : 0.0f;
    m_run = lr_tot > 0.0f ? m_run + __log2f(lr_tot) / c : -INFINITY;
    l_tot *= part_inv;
    lr_tot = lr_tot > 0.0f ? 1.0f : 0.0f;
  };
  if constexpr (PAIR) {
    // Combine the halves: waves 4-7 hand O, the offset m and the sums
    // (normalised as above) to their row partners through LDS, above the
    // rows the epilogue stages; each half's terms are rescaled to the
    // larger offset.
    constexpr int XO = DBLK * 16 * 64;  // floats of O per wave
    static_assert((XO + 4 * 64) * 4 % 1024 == 0 &&
                      256 * D + 4 * (XO + 4 * 64) * 4 <= 8 * T::BYTES,
                  "the combine area (whole KiB per wave) lies inside the ring");
    float* xo = reinterpret_cast<float*>(smem + 256 * D) + rw * (XO + 4 * 64);
    float* xm = xo + XO;
    if (half == 1) {
      if constexpr (kLdsPoison) {
        const uint32_t off = (uint32_t)(reinterpret_cast<char*>(xo) - smem);
        for (int kib = 0; kib < (XO + 4 * 64) * 4 / 1024; ++kib) poison_kib(off + kib * 1024);
        __builtin_amdgcn_s_waitcnt(0xc07f);
      }
#pragma unroll
      for (int db = 0; db < DBLK; ++db)
#pragma unroll
        for (int i = 0; i < 16; ++i) xo[(db * 16 + i) * 64 + lane] = o_acc[db][i];
      *reinterpret_cast<f32x4*>(xm + 4 * lane) = f32x4{m_run, l_tot, lr_tot, 0.0f};
    }
    __syncthreads();
    if (half == 1) return;
    const f32x4 o1 = *reinterpret_cast<const f32x4*>(xm + 4 * lane);
    const float inv1 = o1[2] > 0.0f ? 1.0f / o1[2] : 0.0f;
    const float m1 = o1[2] > 0.0f ? o1[0] + __log2f(o1[2]) / c : -INFINITY;
    normalise_part();
    const float m = fmaxf(m_run, m1);
    const float a0 = m_run == -INFINITY ? 0.0f : fast_exp2((m_run - m) * c);
    const float a1 = m1 == -INFINITY ? 0.0f : fast_exp2((m1 - m) * c);
    const float b0 = a0 * part_inv, b1 = a1 * inv1;
#pragma unroll
    for (int db = 0; db < DBLK; ++db)
#pragma unroll
      for (int i = 0; i < 16; ++i) o_acc[db][i] = o_acc[db][i] * b0 + xo[(db * 16 + i) * 64 + lane] * b1;
    l_tot = l_tot * a0 + o1[1] * b1;
    lr_tot = lr_tot * a0 + (o1[2] > 0.0f ? a1 : 0.0f);
    m_run = m;
  }
  const bool row_ok = qrow < N;
  // The output goes out through LDS, whole rows at a time.  In the O^T
  // accumulator a lane holds 4 consecutive head dims of one row per (db, r),
  // so a direct store instruction writes 32 rows in 8- or 16-byte pieces;
  // staged, each store instruction writes 64 / (row bytes / 16) whole rows
  // with 16 contiguous bytes per lane (+9 % at B4 H16 N1024 D64, +1..2 % at
  // B4 H32 N4096).  The K/V ring is free: the loop ended with a barrier and
  // staged nothing after it.  Each wave uses rows [32 wave, +32) of the ring
  // as an lds::row_tile_offset tile of 32 `rowb`-byte rows, written and
  // read 16 bytes per lane (the LDS serves 8-byte accesses one dword at a
  // time across the wave, so 8-byte pieces would hit even banks only); a
  // wave reads back only what it wrote, so no barrier is needed.
  auto store_rows = [&](int rowb, auto&& put, char* dst, int64_t dst_stride, int rows)
                        FA_INLINE {
    const int nc = rowb >> 4;
    char* ot = smem + wave * 32 * rowb;
    if constexpr (kLdsPoison) {
      for (int kib = 0; kib < rowb / 32; ++kib) poison_kib(wave * 32 * rowb + kib * 1024);
      __builtin_amdgcn_s_waitcnt(0xc07f);
    }
    put([&](int r, int c, auto w) FA_INLINE {
      *reinterpret_cast<decltype(w)*>(ot + lds::row_tile_offset(r, c, rowb)) = w;
    });
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the tile is in LDS
    const int rpi = 64 / nc;             // rows per read
    const int rr = lane / nc, cc = lane & (nc - 1);
#pragma unroll
    for (int j = 0; j < 32 / rpi; ++j) {
      const int r = j * rpi + rr;
      const u32x4 w = *reinterpret_cast<const u32x4*>(ot + lds::row_tile_offset(r, cc, rowb));
      if (r < rows) *reinterpret_cast<u32x4*>(dst + r * dst_stride + cc * 16) = w;
    }
    __builtin_amdgcn_s_waitcnt(0xc07f);  // the reads are done before the ring is reused
  };
  const int wave_rows = max(0, min(32, N - wrow0));  // rows of this wave below N

  if (SPLIT && n_chunks > 1) {
    // ---- split-KV partial, normalised as above: O, offset m' (raw score
    // units; -inf when no key of this chunk is visible to the row), the row
    // sum l for the LSE and the sum of the rounded P (1, or 0 without keys)
    // for the normalisation ----
    normalise_part();
    const int64_t slot =
        (int64_t)args.split.slot[item] + chunk;  // (table items are never chunked)
    const int64_t row0 = ((int64_t)bh * args.split.n_slots + slot) * BM + (wrow0 - q0);
    // fp32 rows of 4D bytes: NW / 4 passes of DBLK / (NW / 4) head-dim
    // blocks each fit the ring (NW x 32 x 4D / passes <= 4 x 64 x 2D).
    constexpr int PASSES = NW / 4, PDB = DBLK / PASSES;
    static_for<0, PASSES>([&](auto p_c) {
      constexpr int p = decltype(p_c)::value;
      store_rows(
          PDB * 128,
          [&](auto&& put) FA_INLINE {
#pragma unroll
            for (int b = 0; b < PDB; ++b)
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                const int db = p * PDB + b;
                const f32x4 w = f32x4{o_acc[db][4 * r + 0], o_acc[db][4 * r + 1],
                                      o_acc[db][4 * r + 2], o_acc[db][4 * r + 3]} * part_inv;
                // cols 32b + 8r + 4g of the pass: chunk 8b + 2r + g
                put(l32, 8 * b + 2 * r + g, w);
              }
          },
          reinterpret_cast<char*>(args.ws_o + row0 * D + p * PDB * 32), int64_t(4 * D), wave_rows);
    });
    if (row_ok && g == 0) {
      const int64_t row = row0 + l32;
      *reinterpret_cast<f32x4*>(args.ws_ml + row * 4) = f32x4{m_run, l_tot, lr_tot, 0.0f};
    }
    return;
  }

  // ---- epilogue: normalise, store ----
  const float inv_l = (row_ok && lr_tot > 0.0f) ? 1.0f / lr_tot : 0.0f;
  store_rows(
      2 * D,
      [&](auto&& put) FA_INLINE {
#pragma unroll
        for (int db = 0; db < DBLK; ++db)
#pragma unroll
          for (int k = 0; k < 2; ++k) {
            // This lane holds 4 columns (half a 16-byte chunk) of row l32 for
            // each of r = 2k and 2k + 1: cols 32db + 8r + 4g .. +3.  One swap
            // of lanes l + 32 <-> l (v_permlane32_swap: the upper half of the
            // first operand with the lower half of the second) leaves lane
            // (l32, g) with the whole chunk 4db + 2k + g of its row.
            const f32x16& o = o_acc[db];
            const int i = 8 * k;
            const u32x2 a = {pack2<BF16>(o[i + 0] * inv_l, o[i + 1] * inv_l),
                             pack2<BF16>(o[i + 2] * inv_l, o[i + 3] * inv_l)};
            const u32x2 b = {pack2<BF16>(o[i + 4] * inv_l, o[i + 5] * inv_l),
                             pack2<BF16>(o[i + 6] * inv_l, o[i + 7] * inv_l)};
            const auto x = __builtin_amdgcn_permlane32_swap(a[0], b[0], false, false);
            const auto y = __builtin_amdgcn_permlane32_swap(a[1], b[1], false, false);
            put(l32, 4 * db + 2 * k + g, u32x4{x[0], y[0], x[1], y[1]});
          }
      },
      oh + wrow0 * osb, osb, wave_rows);
  if (row_ok && args.lse != nullptr && g == 0) {
    const float m_use = m_run == -INFINITY ? 0.0f : m_run;
    args.lse[(int64_t)bh * N + qrow] = m_use * args.scale + __logf(l_tot);
  }
}

// Split-KV merge: one thread per 4 head-dim elements of a row of a q-tile
// with more than one chunk.  O = sum_c w_c O_c / sum_c w_c lr_c with
// w_c = exp2((m_c - m) * c) and m = max_c m_c (the single-pass online
// softmax regrouped by chunk; lr_c is chunk c's sum of the rounded P, and
// chunks whose rows saw no key have l_c = 0 and are skipped),
// LSE = m * scale + ln(sum_c w_c l_c).  Chunks are read kMergeGroup at a
// time with all loads issued together, so a row costs one memory latency
// per group rather than one per chunk.
constexpr int kMergeGroup = 4;

template <int D, bool BF16>
__global__ void __launch_bounds__(256) fa_merge_kernel(const KernelArgs args, int BM) {
  constexpr int TPR = D / 4;       // threads per row
  constexpr int RPB = 256 / TPR;   // rows per workgroup
  const int per_tile = (BM + RPB - 1) / RPB;
  const int per_bh = args.split.n_merge * per_tile;
  const int bh = blockIdx.x / per_bh;
  const int rem = blockIdx.x - bh * per_bh;
  const int mi = rem / per_tile;
  const int r = (rem - mi * per_tile) * RPB + (int)threadIdx.x / TPR;
  const int d = ((int)threadIdx.x % TPR) * 4;
  const uint32_t info = args.split.merge[mi];
  const int qb = (int)(info & 0xffffu);
  const int nch = (int)((info >> 16) & 0xffu);
  const int q = qb * BM + r;
  if (r >= BM || q >= args.seq_len) return;
  // Rows < seq_len of every chunk were written (O = 0, l = 0 where no key
  // was visible), so every load below reads written data.
  const int64_t row0 = ((int64_t)bh * args.split.n_slots + args.split.merge_slot[mi]) * BM + r;
  const float c2 = args.scale_log2;
  float m = -INFINITY, l = 0.0f, lr = 0.0f;
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  for (int c0 = 0; c0 < nch; c0 += kMergeGroup) {
    f32x4 ml[kMergeGroup];  // (m, l, lr, unused)
    f32x4 oc[kMergeGroup];
#pragma unroll
    for (int j = 0; j < kMergeGroup; ++j) {
      const int64_t rc = row0 + (int64_t)min(c0 + j, nch - 1) * BM;
      ml[j] = *reinterpret_cast<const f32x4*>(args.ws_ml + rc * 4);
      oc[j] = *reinterpret_cast<const f32x4*>(args.ws_o + rc * D + d);
    }
    float mg = m;
#pragma unroll
    for (int j = 0; j < kMergeGroup; ++j)
      if (c0 + j < nch && ml[j][1] > 0.0f) mg = fmaxf(mg, ml[j][0]);
    if (l > 0.0f && mg > m) {
      const float a = fast_exp2((m - mg) * c2);
      l *= a;
      lr *= a;
      acc *= a;
    }
    m = mg;
#pragma unroll
    for (int j = 0; j < kMergeGroup; ++j)
      if (c0 + j < nch && ml[j][1] > 0.0f) {
        const float w = fast_exp2((ml[j][0] - m) * c2);
        l += w * ml[j][1];
        lr += w * ml[j][2];
        acc += w * oc[j];
      }
  }
  const float inv_l = lr > 0.0f ? 1.0f / lr : 0.0f;
  const int b = bh / args.heads;
  const int h = bh - b * args.heads;
  char* op = reinterpret_cast<char*>(args.o) +
             2 * (b * args.o_stride_b + h * args.o_stride_h + (int64_t)q * args.o_stride_s + d);
  *reinterpret_cast<u32x2*>(op) = u32x2{pack2<BF16>(acc[0] * inv_l, acc[1] * inv_l),
                                        pack2<BF16>(acc[2] * inv_l, acc[3] * inv_l)};
  if (args.lse != nullptr && d == 0)
    args.lse[(int64_t)bh * args.seq_len + q] = (m == -INFINITY ? 0.0f : m) * args.scale + __logf(l);
}

template <int D, bool BF16, bool CAUSAL, int NW, bool PAIR = false>
hipError_t launch_one(const KernelArgs& a, hipStream_t stream) {
  constexpr int BM = PAIR ? 128 : 32 * NW;
  KernelArgs args = a;
  // Pair mode runs one workgroup per q-tile, longest first; its plan has no items.
  if (PAIR && (a.split.n_items != 0 || !CAUSAL)) return hipErrorInvalidValue;
  args.n_qblocks = (args.seq_len + BM - 1) / BM;
  // A plan is only valid for the block height it was made for; partials
  // need the workspace; a placement table covers 8 XCDs of whole heads.
  const int64_t bh = (int64_t)args.batch * args.heads;
  const SplitPlan& sp = args.split;
  if (sp.n_items > 0 &&
      (block_rows(args) != BM || sp.n_items > kMaxSplitItems ||
       (sp.n_merge > 0 && (args.ws_o == nullptr || args.ws_ml == nullptr)) ||
       (sp.xcd_heads > 0 && bh != 8 * (int64_t)sp.xcd_heads)))
    return hipErrorInvalidValue;
  const int64_t total = sp.xcd_heads > 0 ? 8 * (int64_t)sp.n_items
                                         : (sp.n_items > 0 ? sp.n_items : args.n_qblocks) * bh;
  if (total > 0x7fffffff) return hipErrorInvalidValue;
  // hipLaunchKernel returns this launch's own status: the thread's last-error
  // state is neither read nor cleared, so an earlier failure of an unrelated
  // HIP call by the caller is not reported as (or lost to) this launch.
  void* kargs[] = {&args};
  // bf16 pair and split launches that write an LSE: the LSE_L form, whose
  // optimistic pass keeps the unrounded sums.
  const bool lse_l = BF16 && args.lse != nullptr;
  if (args.split.n_items == 0) {
    const void* fn = reinterpret_cast<const void*>(&fa_fwd_kernel<D, BF16, CAUSAL, NW, false, PAIR>);
    if constexpr (BF16 && PAIR)
      if (lse_l) fn = reinterpret_cast<const void*>(&fa_fwd_kernel<D, BF16, CAUSAL, NW, false, PAIR, true>);
    return hipLaunchKernel(fn, dim3((unsigned)total), dim3(NW * 64), kargs, 0, stream);
  }
  if constexpr (PAIR) {
    return hipErrorInvalidValue;  // (rejected above: pair plans have no items)
  } else {
    const void* fn = reinterpret_cast<const void*>(&fa_fwd_kernel<D, BF16, CAUSAL, NW, true>);
    if constexpr (BF16)
      if (lse_l) fn = reinterpret_cast<const void*>(&fa_fwd_kernel<D, BF16, CAUSAL, NW, true, false, true>);
    hipError_t e = hipLaunchKernel(fn, dim3((unsigned)total), dim3(NW * 64), kargs, 0, stream);
    if (e != hipSuccess || sp.n_merge == 0) return e;
    constexpr int RPB = 256 / (D / 4);
    const int64_t merge_blocks = bh * args.split.n_merge * ((BM + RPB - 1) / RPB);
    if (merge_blocks > 0x7fffffff) return hipErrorInvalidValue;
    int bm = BM;
    void* margs[] = {&args, &bm};
    return hipLaunchKernel(reinterpret_cast<const void*>(&fa_merge_kernel<D, BF16>),
                           dim3((unsigned)merge_blocks), dim3(256), margs, 0, stream);
  }
}

// The 16x16x32 MFMA kernel of every unsplit launch outside pair mode.
#include "fa_fwd16.inc"

// fa_fwd16_kernel where it runs (see launch_causal), else fa_fwd_kernel.
template <int D, bool BF16, bool CAUSAL, int NW>
hipError_t launch_pick(const KernelArgs& a, hipStream_t stream, bool plain) {
#ifndef FA_MFMA32
  if constexpr (D == 128 || BF16 || CAUSAL || NW == 8)
    if (plain) return launch16<D, BF16, CAUSAL, NW>(a, stream);
#endif
  return launch_one<D, BF16, CAUSAL, NW>(a, stream);
}

template <int D, bool BF16>
hipError_t launch_causal(const KernelArgs& a, hipStream_t stream) {
  // Launches without split-KV chunks or pair mode (plain order or an XCD
  // placement table) run fa_fwd16_kernel, the 16x16x32 MFMA form, except
  // fp16 non-causal 4-wave grids at D = 64; split chunks, pair mode and those
  // run this file's 32x32x16 kernel.  Measured on two boxes, 16x16x32
  // against 32x32x16: +2...+8 % at B4 H32 N4096 fp16, +2...+4 % at bf16
  // causal B2 H32 N8192, +0...+5 % on fp16 causal B1 H16 N16384.  At D = 64
  // (same box): fp16 non-causal 4-wave B4 H16 N1024 -0.3 % (-1.5 % with
  // Q, K ~ N(0, 3^2)), B3 H16 N1024 -4 %, where the softmax's VALU work
  // matches the MFMA work and the 16x16 shape takes twice the MFMA issue
  // slots; but 8-wave B2 H16 N4096 +4.4 % (bf16 +13 %), bf16 B4 H16 N1024
  // +15 %, causal B2 H16 N4096 +15 % (bf16 +20 %), the causal placement
  // table B1 H16 N4096 +9 % (bf16 +15 %), causal B1 H16 N16384 with
  // Q, K ~ N(0, 3^2) +2.7 %.  The test-only build
  // libfa_mi355x_mfma32.so (-DFA_MFMA32) runs the 32x32x16 kernel
  // everywhere, for the counter comparison of the two shapes.
  const bool plain =
      a.split.n_items == 0 || (a.split.xcd_heads > 0 && a.split.n_merge == 0);
  if (a.causal) {
    // Long causal rows: 8-wave workgroups (fp16: +1.4 % at B1 H16 N16384,
    // +4 % with the matrix-core row sums they enable; bf16 only where the
    // 4-wave grid would be split, block_rows); short problems lose (-11 % at N = 3000: fewer,
    // longer workgroups).
    if (block_rows(a) == 256) return launch_pick<D, BF16, true, 8>(a, stream, plain);
    // Grids of 0.75 to 2 q-tiles per CU: pair mode (plan_split decides).
    if (a.split.pair) return launch_one<D, BF16, true, 8, true>(a, stream);
    return launch_pick<D, BF16, true, 4>(a, stream, plain);
  }
  // Long non-causal rows: 8 waves (BM = 256) per workgroup, one workgroup
  // per CU, halve the L2->LDS tile traffic per flop; the chip is power
  // limited there and the saved data movement buys clock (measured +3 % at
  // N = 4096).  Shorter or causal problems keep 4 waves and two workgroups
  // per CU, which fill the machine better.
  const bool plain_nc = a.split.n_items == 0;
  if (a.seq_len >= kWideMinSeq)
    return launch_pick<D, BF16, false, 8>(a, stream, plain_nc);
  return launch_pick<D, BF16, false, 4>(a, stream, plain_nc);
}

}  // namespace

hipError_t scratch_buffer(void** ptr) {
  // Device address of `scratch` on each device, looked up once per device
  // (with that device current) and kept.
  constexpr int kMaxDevices = 64;
  static std::atomic<void*> addr[kMaxDevices];
  static std::mutex lock;
  *ptr = nullptr;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  void* p = addr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    std::lock_guard<std::mutex> g(lock);
    p = addr[dev].load(std::memory_order_acquire);
    if (p == nullptr) {
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess) return e;
      if (p == nullptr) return hipErrorInvalidSymbol;
      addr[dev].store(p, std::memory_order_release);
    }
  }
  *ptr = p;
  return hipSuccess;
}

hipError_t launch_fwd(const KernelArgs& a, hipStream_t stream) {
  if (a.head_dim == 128)
    return a.bf16 ? launch_causal<128, true>(a, stream) : launch_causal<128, false>(a, stream);
  return a.bf16 ? launch_causal<64, true>(a, stream) : launch_causal<64, false>(a, stream);
}

}  // namespace fa
