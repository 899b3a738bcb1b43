// Host build of the kernel's LDS layout functions (flash-attention_amd/csrc/
// fa_lds_layout.h) for the CPU layout checks in tests/test_lds_layout.py.
// Test infrastructure: never linked into the library.
#include "fa_lds_layout.h"

namespace {

template <int D, int NW, bool IS_V>
int dma_map(int* r, int* c) {
  constexpr int ITERS = fa::lds::Tile<D>::BYTES / (1024 * NW);
  int n = 0;
  for (int w = 0; w < NW; ++w)
    for (int it = 0; it < ITERS; ++it)
      for (int lane = 0; lane < 64; ++lane, ++n) fa::lds::dma_slot<D, NW, IS_V>(w, it, lane, r[n], c[n]);
  return n;
}

template <int D>
int k_reads(int* off) {
  int n = 0;
  for (int kb = 0; kb < 2; ++kb)
    for (int kk = 0; kk < D / 16; ++kk)
      for (int lane = 0; lane < 64; ++lane) off[n++] = fa::lds::k_read_offset<D>(kb, kk, lane);
  return n;
}

template <int D>
int v_reads(int* off) {
  int n = 0;
  for (int ch = 0; ch < 4; ++ch)
    for (int hf = 0; hf < 2; ++hf)
      for (int db = 0; db < D / 32; ++db)
        for (int lane = 0; lane < 64; ++lane) off[n++] = fa::lds::v_read_offset<D>(ch, hf, db, lane);
  return n;
}

template <int D, int NW, bool IS_V>
int dma_map16(int* r, int* c) {
  constexpr int ITERS = fa::lds::Tile<D>::BYTES / (1024 * NW);
  int n = 0;
  for (int w = 0; w < NW; ++w)
    for (int it = 0; it < ITERS; ++it)
      for (int lane = 0; lane < 64; ++lane, ++n) fa::lds::dma_slot16<D, NW, IS_V>(w, it, lane, r[n], c[n]);
  return n;
}

template <int D>
int k16_reads(int* off) {
  int n = 0;
  for (int kb = 0; kb < 4; ++kb)
    for (int st = 0; st < D / 32; ++st)
      for (int lane = 0; lane < 64; ++lane) off[n++] = fa::lds::k16_read_offset<D>(kb, st, lane);
  return n;
}

template <int D>
int v16_reads(int* off) {
  int n = 0;
  for (int ch = 0; ch < 2; ++ch)
    for (int h = 0; h < 2; ++h)
      for (int db = 0; db < D / 16; ++db)
        for (int lane = 0; lane < 64; ++lane) off[n++] = fa::lds::v16_read_offset<D>(ch, h, db, lane);
  return n;
}

}  // namespace

extern "C" {

// The 16x16x32 kernel's layout (lds::Tile16): DMA map as fa_lds_dma_map, K
// operand offsets [kb 4][st D/32][lane 64], V^T offsets [ch 2][h 2][db D/16][lane 64].
int fa_lds_dma_map16(int D, int NW, int is_v, int* r, int* c) {
  if (D == 128 && NW == 4) return is_v ? dma_map16<128, 4, true>(r, c) : dma_map16<128, 4, false>(r, c);
  if (D == 128 && NW == 8) return is_v ? dma_map16<128, 8, true>(r, c) : dma_map16<128, 8, false>(r, c);
  if (D == 64 && NW == 4) return is_v ? dma_map16<64, 4, true>(r, c) : dma_map16<64, 4, false>(r, c);
  if (D == 64 && NW == 8) return is_v ? dma_map16<64, 8, true>(r, c) : dma_map16<64, 8, false>(r, c);
  return -1;
}
int fa_lds_k16_reads(int D, int* off) {
  return D == 128 ? k16_reads<128>(off) : D == 64 ? k16_reads<64>(off) : -1;
}
int fa_lds_v16_reads(int D, int* off) {
  return D == 128 ? v16_reads<128>(off) : D == 64 ? v16_reads<64>(off) : -1;
}

// (row, logical chunk) fetched by DMA lane (wave, it, lane), in that order;
// returns the number of entries (NW * ITERS * 64) or -1 for an unknown shape.
int fa_lds_dma_map(int D, int NW, int is_v, int* r, int* c) {
  if (D == 128 && NW == 4) return is_v ? dma_map<128, 4, true>(r, c) : dma_map<128, 4, false>(r, c);
  if (D == 128 && NW == 8) return is_v ? dma_map<128, 8, true>(r, c) : dma_map<128, 8, false>(r, c);
  if (D == 64 && NW == 4) return is_v ? dma_map<64, 4, true>(r, c) : dma_map<64, 4, false>(r, c);
  if (D == 64 && NW == 8) return is_v ? dma_map<64, 8, true>(r, c) : dma_map<64, 8, false>(r, c);
  return -1;
}

// K operand read offsets [kb 2][kk D/16][lane 64].
int fa_lds_k_reads(int D, int* off) {
  return D == 128 ? k_reads<128>(off) : D == 64 ? k_reads<64>(off) : -1;
}

// V^T operand read offsets [ch 4][hf 2][db D/32][lane 64].
int fa_lds_v_reads(int D, int* off) {
  return D == 128 ? v_reads<128>(off) : D == 64 ? v_reads<64>(off) : -1;
}

// Row tiles: byte offset of (row r, chunk c) in a 32-row tile of rowb-byte rows.
int fa_lds_row_offset(int r, int c, int rowb) { return fa::lds::row_tile_offset(r, c, rowb); }

}  // extern "C"
