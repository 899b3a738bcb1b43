// LDS layout of the K and V tiles of the forward kernel: where the staging
// DMA puts each lane's 16 bytes, the XOR swizzles, and the byte offsets the
// MFMA operand reads use.  Shared by the kernel (fa_fwd_kernel.hip, device
// code) and the CPU layout checks (tests/lds/, host code), so the checks run
// the same functions the kernel runs.
//
// Replaces the reference's smem layout (src/loadstore/copy_gsm.cuh:31-47
// smem_offset_g2s, src/loadstore/copy_srm.cuh:14-30 smem_offset,
// src/tensor_core/swizzle.cuh:5-28 Swizzle<3,3,3>), which is built for 32-bank
// NVIDIA shared memory and ldmatrix; this one is derived for the gfx950 LDS
// and the reads below.
#pragma once

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define FA_LAYOUT_FN __host__ __device__ __forceinline__
#else
#define FA_LAYOUT_FN inline
#endif

// Bits cleared from the K / V swizzles.  Always 0 in the library; the CPU
// layout checks build a copy with one bit cleared to show they detect it.
#ifndef FA_LDS_SWZ_K_CLEAR
#define FA_LDS_SWZ_K_CLEAR 0
#endif
#ifndef FA_LDS_SWZ_V_CLEAR
#define FA_LDS_SWZ_V_CLEAR 0
#endif
// The same for the row tiles: bits cleared from row_swz.
#ifndef FA_LDS_ROW_SWZ_CLEAR
#define FA_LDS_ROW_SWZ_CLEAR 0
#endif

namespace fa {
namespace lds {

template <int D>
struct Tile {
  static constexpr int BN = 64;            // keys per K/V tile
  static constexpr int ROWB = D * 2;       // bytes per K/V row
  static constexpr int BYTES = BN * ROWB;  // bytes per K or V tile
  // K tile: the 32x32x16 A-operand read is ds_read_b128 of one 16-byte chunk
  // per lane for 32 consecutive keys; XOR the chunk index with key bits so
  // consecutive keys land on distinct bank groups.
  static FA_LAYOUT_FN int swz_k(int key) {
    return (D == 128 ? (key & 15) : ((key >> 1) & 7)) & ~FA_LDS_SWZ_K_CLEAR;
  }
  // V tile: a transposed read covers 4 consecutive keys x 64 contiguous bytes
  // per half-wave; XOR the 64-byte segment so the 4 keys hit distinct banks.
  static FA_LAYOUT_FN int swz_v(int key) {
    return (D == 128 ? ((key & 3) << 2) : (((key >> 1) & 1) << 2)) & ~FA_LDS_SWZ_V_CLEAR;
  }
};

// Where lane `lane` of wave `wave` lands in a K/V LDS tile for DMA
// instruction `it`: tile row r and the logical 16-byte chunk it must fetch.
// The LDS destination of a DMA lane is fixed at base + 16*lane (the
// instruction's base is byte (wave*ITERS + it)*1024 of the tile), so the XOR
// swizzle is applied to the source chunk instead.
template <int D, int NW, bool IS_V>
FA_LAYOUT_FN void dma_slot(int wave, int it, int lane, int& r, int& c) {
  using T = Tile<D>;
  constexpr int ITERS = T::BYTES / (1024 * NW);
  const int off = (wave * ITERS + it) * 1024 + lane * 16;
  r = off / T::ROWB;
  const int pc = (off % T::ROWB) / 16;
  c = pc ^ (IS_V ? T::swz_v(r) : T::swz_k(r));
}

// Byte offset within a K tile of the 16 bytes lane `lane` reads (one
// ds_read_b128) as the A operand of S^T = K Q^T for key block kb (32 keys)
// and k-step kk: key kb*32 + lane%32, head dims [16kk + 8(lane/32), +8).
// Keys of block 1 sit 32 rows below block 0 with the same swizzle bits, so
// the kernel adds kb*32*ROWB to the block-0 offset.
template <int D>
FA_LAYOUT_FN int k_read_offset(int kb, int kk, int lane) {
  using T = Tile<D>;
  const int key = kb * 32 + (lane & 31);
  const int chunk = 2 * kk + (lane >> 5);
  return key * T::ROWB + ((chunk ^ T::swz_k(key)) << 4);
}

// Byte offset within a V tile of the 8 bytes lane `lane` addresses with one
// ds_read_b64_tr_b16 for the V^T operand of 16-key chunk ch, half hf and
// 32-wide head-dim block db.  The lane supplies row key = 16ch + 8hf +
// 4(lane/32) + (lane%16)/4 and columns 32db + 16((lane/16)%2) + 4(lane%4) ..
// +3 (the transposing read hands lane i of each 16-lane group element i%4
// of the words addressed by lanes 4e + i/4).  Multiples of 4 keys keep the
// swizzle bits, so the kernel adds ch*16*ROWB + hf*8*ROWB as immediates.
template <int D>
FA_LAYOUT_FN int v_read_offset(int ch, int hf, int db, int lane) {
  using T = Tile<D>;
  const int lj = lane & 15, hg = (lane >> 4) & 1, g = lane >> 5;
  const int key = 16 * ch + 8 * hf + 4 * g + (lj >> 2);
  const int col = 32 * db + 16 * hg + 4 * (lj & 3);
  return key * T::ROWB + (((col >> 3) ^ T::swz_v(key)) << 4) + (col & 7) * 2;
}

// ---- Layout of the 16x16x32 kernel (fa_fwd16_kernel) ----
// K tiles keep Tile<D>::swz_k: its 16-byte reads cover 16 consecutive keys
// (lanes l % 16) of one chunk, which the swizzle spreads over all 64 banks.
// V tiles get their own chunk swizzle: a 32-lane pass of the transposing
// read covers 8 consecutive keys x 32 bytes (two chunks of head dims), so
// each key's chunk pair is XORed with a distinct even index.  Both swizzles
// only depend on key % 16, so key blocks 16 apart share the per-lane offsets.
#ifndef FA_LDS_SWZ_V16_CLEAR
#define FA_LDS_SWZ_V16_CLEAR 0
#endif
template <int D>
struct Tile16 {
  static FA_LAYOUT_FN int swz_k(int key) { return Tile<D>::swz_k(key); }
  static FA_LAYOUT_FN int swz_v(int key) {
    return (D == 128 ? ((key & 7) << 1) : (((key >> 1) & 3) << 1)) & ~FA_LDS_SWZ_V16_CLEAR;
  }
};

// DMA placement (as dma_slot) with the 16x16 kernel's V swizzle.
template <int D, int NW, bool IS_V>
FA_LAYOUT_FN void dma_slot16(int wave, int it, int lane, int& r, int& c) {
  using T = Tile<D>;
  constexpr int ITERS = T::BYTES / (1024 * NW);
  const int off = (wave * ITERS + it) * 1024 + lane * 16;
  r = off / T::ROWB;
  const int pc = (off % T::ROWB) / 16;
  c = pc ^ (IS_V ? Tile16<D>::swz_v(r) : Tile16<D>::swz_k(r));
}

// Byte offset within a K tile of the 16 bytes lane `lane` reads (one
// ds_read_b128) as the A operand of the 16x16x32 S^T product for key block
// kb (16 keys) and k-step st (32 head dims): key 16kb + lane % 16, head dims
// [32st + 8(lane / 16), +8).  Key block kb adds kb * 16 * ROWB to block 0.
template <int D>
FA_LAYOUT_FN int k16_read_offset(int kb, int st, int lane) {
  using T = Tile<D>;
  const int key = 16 * kb + (lane & 15);
  const int chunk = 4 * st + (lane >> 4);
  return key * T::ROWB + ((chunk ^ Tile16<D>::swz_k(key)) << 4);
}

// Byte offset within a V tile of the 8 bytes lane `lane` addresses with one
// ds_read_b64_tr_b16 for the V^T operand of 32-key chunk ch, half h and
// 16-wide head-dim block db: row key = 32ch + 16h + 4(lane / 16) +
// (lane % 16) / 4, columns 16db + 4(lane % 4) .. +3 (the transposing read
// hands lane i of each 16-lane group element i % 4 of the words addressed
// by lanes 4e + i / 4, so lane i of group g receives V[32ch + 16h + 4g + e]
// [16db + i] for e = 0..3).  Chunks and halves add (32ch + 16h) * ROWB.
template <int D>
FA_LAYOUT_FN int v16_read_offset(int ch, int h, int db, int lane) {
  using T = Tile<D>;
  const int l16 = lane & 15, g4 = lane >> 4;
  const int key = 32 * ch + 16 * h + 4 * g4 + (l16 >> 2);
  const int col = 16 * db + 4 * (l16 & 3);
  return key * T::ROWB + (((col >> 3) ^ Tile16<D>::swz_v(key)) << 4) + (col & 7) * 2;
}

// Row tiles: 32 rows of `rowb` bytes (rowb = 128, 256 or 512) that a wave
// stages on its own, Q for its MFMA operands (4-wave workgroups) and O or
// the fp32 split partials on their way out.  Row r's 16-byte chunk c sits at
// chunk position c ^ row_swz(r).  The writes put one chunk per lane over 32
// rows (lane l: row l % 32); a ds_write_b128 serves 8 lanes per LDS cycle,
// which conflict unless their chunks differ mod 128 bytes, so each aligned
// group of 8 rows needs 8 distinct positions mod 128.  The 16-byte reads
// serve 16 lanes per cycle over all 256 bytes of banks: whole rows, and for
// Q one chunk of 16 consecutive rows, which at rowb = 128 needs the even
// and the odd rows of the 16 on distinct positions.  rowb >= 256: r mod
// the row's chunk count; rowb = 128: r ^ (r >> 3) mod 8.
FA_LAYOUT_FN int row_swz(int r, int rowb) {
  const int nc = rowb >> 4;  // chunks per row
  return (nc >= 16 ? (r & (nc - 1)) : ((r ^ (r >> 3)) & (nc - 1))) & ~FA_LDS_ROW_SWZ_CLEAR;
}
FA_LAYOUT_FN int row_tile_offset(int r, int c, int rowb) {
  return r * rowb + ((c ^ row_swz(r, rowb)) << 4);
}

}  // namespace lds
}  // namespace fa
