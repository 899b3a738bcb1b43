// LDS bank-conflict probe for gfx950: one dispatch per access pattern, each
// wave issuing the pattern's LDS instruction 64 times at fixed per-lane
// offsets (all inside the workgroup's 64 KiB), so that SQ_LDS_BANK_CONFLICT /
// SQ_INSTS_LDS of a dispatch is the conflict cycles of one instruction.
// The measured values calibrate the bank model of tests/test_lds_layout.py,
// which recomputes the same offsets (kPatterns there lists them in the same
// order).  Build and count (from the repository root):
//   hipcc --offload-arch=gfx950 -O3 -std=c++17 -Xclang -target-feature \
//     -Xclang -packed-fp32-ops -I flash-attention_amd/csrc \
//     tests/lds/lds_bank_probe.hip -o /tmp/lds_bank_probe
//   rocprofv3 --pmc SQ_LDS_BANK_CONFLICT SQ_INSTS_LDS SQ_LDS_IDX_ACTIVE SQ_WAVES \
//     --output-format csv -d <dir> -o c -- /tmp/lds_bank_probe
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <utility>

#include "fa_lds_layout.h"

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4_t;
typedef __attribute__((address_space(3))) volatile u32x4 lds_u32x4_t;
typedef __attribute__((address_space(3))) char lds_char;

enum Kind { kRead128 = 0, kWrite128 = 1, kReadTr64 = 2 };

// The row tile of 128-byte rows before the current swizzle: chunk c of row r
// at c ^ ((r >> 1) & 7).
__host__ __device__ int old_row128(int r, int c) { return r * 128 + ((c ^ ((r >> 1) & 7)) << 4); }

template <int P>
__device__ __forceinline__ int offset_of(int lane, Kind& kind) {
  const int l32 = lane & 31, g = lane >> 5;
  namespace L = fa::lds;
  kind = kRead128;
  switch (P) {
    case 0: return lane * 16;                                   // linear read
    case 1: return lane * 256;                                  // every lane of a pass on one bank group
    case 2: kind = kWrite128; return old_row128(l32, 0 + g);    // O staging, D = 64, old swizzle
    case 3: kind = kWrite128; return old_row128(l32, 2 + g);
    case 4: kind = kWrite128; return old_row128(l32, 4 + g);
    case 5: kind = kWrite128; return old_row128(l32, 6 + g);
    case 6: return old_row128(lane / 8, lane & 7);              // whole-row reads, old swizzle
    case 7: return old_row128(8 + lane / 8, lane & 7);
    case 8: return old_row128(l32, 0 + g);                      // Q operand reads, old swizzle
    case 9: return old_row128(l32, 2 + g);
    case 10: kind = kWrite128; return L::row_tile_offset(l32, 0 + g, 256);
    case 11: return L::row_tile_offset(lane / 16, lane & 15, 256);
    case 12: return L::k_read_offset<64>(0, 0, lane);
    case 13: return L::k_read_offset<64>(0, 1, lane);
    case 14: kind = kReadTr64; return L::v_read_offset<64>(0, 0, 0, lane);
    case 15: kind = kReadTr64; return L::v_read_offset<64>(0, 0, 1, lane);
    case 16: kind = kWrite128; return lane * 16;                // linear write
    case 17: kind = kWrite128; return lane * 256;
    case 18: return L::k_read_offset<128>(0, 0, lane);
    case 19: kind = kReadTr64; return L::v_read_offset<128>(0, 0, 0, lane);
    case 20: kind = kWrite128; return L::row_tile_offset(l32, 2 + g, 256);
    case 21: return L::row_tile_offset(l32, 0 + g, 256);
    case 22: kind = kWrite128; return (lane & 15) * 16 + (lane >> 4) * 1024;
    case 23: kind = kWrite128; return l32 * 16 + g * 8192;      // lanes l and l + 32 on one bank group
    case 24: return l32 * 16 + g * 8192;
    case 25: kind = kWrite128; return (lane & 7) * 16 + ((lane >> 3) & 1) * 8192 + (lane >> 4) * 128;
    case 26: kind = kWrite128; return L::row_tile_offset(l32, 0 + g, 128);  // current swizzle
    case 27: kind = kWrite128; return L::row_tile_offset(l32, 6 + g, 128);
    case 28: return L::row_tile_offset(lane / 8, lane & 7, 128);
    case 29: return L::row_tile_offset(l32, 0 + g, 128);
    case 30: return L::row_tile_offset(l32, 6 + g, 128);
    default: return 0;
  }
}

constexpr int kNumPatterns = 31;

template <int P>
__global__ void __launch_bounds__(256) lds_probe(uint32_t* out) {
  __shared__ __attribute__((aligned(1024))) char smem[65536];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  Kind kind;
  // each wave on its own 16 KiB (patterns span at most 16 KiB)
  const int off = offset_of<P>(lane, kind) + (wave & 3) * 16384;
  lds_char* base = (lds_char*)(smem);
  u32x4 acc = {0, 0, 0, 0};
  if (kind == kWrite128) {
    lds_u32x4_t* p = (lds_u32x4_t*)(base + off);
#pragma unroll 1
    for (int i = 0; i < 64; ++i) *p = u32x4{(uint32_t)i, 1u, 2u, 3u};
  } else if (kind == kRead128) {
    lds_u32x4_t* p = (lds_u32x4_t*)(base + off);
#pragma unroll 1
    for (int i = 0; i < 64; ++i) acc ^= *p;
  } else {
    lds_i16x4_t* q = (lds_i16x4_t*)(base + off);
#pragma unroll 1
    for (int i = 0; i < 64; ++i) {
      const i16x4 x = __builtin_amdgcn_ds_read_tr16_b64_v4i16(q);
      acc[0] ^= (uint32_t)(unsigned short)x[0] ^ ((uint32_t)(unsigned short)x[3] << 16);
      asm volatile("" : "+v"(acc));
    }
  }
  out[blockIdx.x * 256 + threadIdx.x] = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
}

template <int P>
void launch(uint32_t* d) {
  hipLaunchKernelGGL(lds_probe<P>, dim3(256), dim3(256), 0, 0, d);
  const hipError_t e = hipDeviceSynchronize();
  if (e != hipSuccess) {
    std::fprintf(stderr, "pattern %d: %s\n", P, hipGetErrorString(e));
    std::exit(1);
  }
}

template <int... Ps>
void launch_all(uint32_t* d, std::integer_sequence<int, Ps...>) {
  (launch<Ps>(d), ...);
}

}  // namespace

int main() {
  uint32_t* d = nullptr;
  if (hipMalloc(&d, 256 * 256 * sizeof(uint32_t)) != hipSuccess) return 1;
  launch_all(d, std::make_integer_sequence<int, kNumPatterns>{});
  std::printf("lds_bank_probe: %d patterns done\n", kNumPatterns);
  return hipFree(d) == hipSuccess ? 0 : 1;
}
