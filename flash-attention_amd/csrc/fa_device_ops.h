// Device building blocks of the MI355X (gfx950) FlashAttention-2 forward:
// MFMA wrappers, packed conversions, cross-half-wave reductions, the
// transposing LDS read and the direct global->LDS DMA.  Shared by the kernel
// (fa_fwd_kernel.hip) and the known-answer tests (tests/kat/fa_kat.hip),
// which check each of them on the GPU.
//
// These replace the reference's ISA wrappers (src/ptx/mma_atom.cuh:8-31,
// src/ptx/ptx.cuh:9-126, src/ptx/copy.cuh:14-79) and the quad-shuffle
// reductions of src/softmax/online_softmax.cuh:21-31 with their CDNA4
// counterparts; they are not translations of them.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

// Kernel-local lambdas carry this so they are always inlined: an outlined
// lambda receives its by-reference captures through scratch memory.
#define FA_INLINE __attribute__((always_inline))

namespace fa {
namespace dev {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(3))) i16x4 lds_i16x4_t;
typedef __attribute__((address_space(3))) i16x8 lds_i16x8_t;

constexpr int kNumXcd = 8;  // MI355X: 8 XCDs, blocks dispatched round-robin

template <bool BF16>
struct ElemOps;

template <>
struct ElemOps<false> {
  using scalar = _Float16;
  static __device__ __forceinline__ f32x16 mfma(i16x8 a, i16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                 __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
};

template <>
struct ElemOps<true> {
  using scalar = __bf16;
  static __device__ __forceinline__ f32x16 mfma(i16x8 a, i16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                  __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
};

// Two fp32 -> packed pair of the element type, round-to-nearest-even
// (one v_cvt_pk_f16_f32 / v_cvt_pk_bf16_f32).
template <bool BF16>
__device__ __forceinline__ uint32_t pack2(float x, float y) {
  const f32x2 f = {x, y};
  if constexpr (BF16) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, bf16x2));
  } else {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f, f16x2));
  }
}

// acc + lo(w) + hi(w) for a packed pair w of the element type, accumulated in
// fp32 (v_dot2c_f32_f16 / v_dot2c_f32_bf16 against (1, 1)).
template <bool BF16>
__device__ __forceinline__ float dot2_acc(uint32_t w, float acc) {
  if constexpr (BF16) {
    const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, w), one, acc, false);
  } else {
    const f16x2 one = {(_Float16)1.0f, (_Float16)1.0f};
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, w), one, acc, false);
  }
}

// Row sums of P on the matrix core.  A P^T chunk register (the B operand of
// the 32x32x16 PV product: lane l holds 8 keys of query row l % 32, key half
// l / 32) read as the B operand of v_mfma_f32_16x16x32_{f16,bf16} has
// B[k = 8*(l/16) + j][n = l % 16]: k-groups 0 and 2 are rows 0..15, groups
// 1 and 3 rows 16..31.  With the selector A (row 0 = ones on k-groups 0 and 2,
// row 1 = ones on groups 1 and 3, other rows 0) the product adds the chunk's
// 16-key sum of row n to C[0][n] and of row n + 16 to C[1][n]; lane n < 16
// holds C[0][n] in element 0 and C[1][n] in element 1 (every other element
// of the accumulator stays 0).
template <bool BF16>
__device__ __forceinline__ i16x8 row_sum_selector(int lane) {
  const short one = BF16 ? (short)0x3F80 : (short)0x3C00;  // 1.0 in bf16 / fp16
  const short v = ((lane & 15) == ((lane >> 4) & 1)) ? one : (short)0;
  return i16x8{v, v, v, v, v, v, v, v};
}
template <bool BF16>
__device__ __forceinline__ f32x4 row_sum_mfma(i16x8 sel, i16x8 p, f32x4 acc) {
  if constexpr (BF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, sel),
                                                   __builtin_bit_cast(bf16x8, p), acc, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, sel),
                                                  __builtin_bit_cast(f16x8, p), acc, 0, 0, 0);
  }
}
// Scale the row sums by a per-row factor held, like every per-row value of
// the S^T layout, by lane l for row l % 32 (all lanes active).
__device__ __forceinline__ f32x4 row_sum_scale(f32x4 acc, float f, int lane) {
  const float f_hi = __shfl(f, (lane & 15) + 16);  // row n + 16's factor, for lane n
  acc[0] *= f;
  acc[1] *= f_hi;
  return acc;
}
// The accumulated sum of lane `lane`'s query row (row lane % 32).
__device__ __forceinline__ float row_sum_of_lane(f32x4 acc, int lane) {
  const float lo = __shfl(acc[0], lane & 15);
  const float hi = __shfl(acc[1], lane & 15);
  return (lane & 31) < 16 ? lo : hi;
}

// Compile-time loop: f(std::integral_constant<int, I>) for I in [B, E).
template <int B, int E, class F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Lanes l and l^32 hold the two halves of one query row.  After
// v_permlane32_swap vdst, src0 (both holding x) vdst = x[l % 32] and
// src0 = x[l % 32 + 32] in every lane l; combine them.  Issued from inline
// asm because the compiler's two-result builtin returns the same register
// for both results; s_nop 1 provides the two wait states the instruction
// needs after a VALU write of its operands.
__device__ __forceinline__ void pair_values(float x, float& lo, float& hi) {
  uint32_t a = __builtin_bit_cast(uint32_t, x);
  uint32_t b = a;
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
  lo = __builtin_bit_cast(float, a);
  hi = __builtin_bit_cast(float, b);
}
// max(a, b, c) in one v_max3_f32.  Issued from inline asm because fmaxf
// makes the compiler quiet possible signalling NaNs with an extra v_max of
// each MFMA result first; the scores here are never NaN.
__device__ __forceinline__ float max3(float a, float b, float c) {
  float d;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(d) : "v"(a), "v"(b), "v"(c));
  return d;
}
// Max over lanes l and l^32 (v_max3 with a repeated operand: no
// canonicalising v_max of the inputs, which fmaxf would add).
__device__ __forceinline__ float pair_max(float x) {
  float lo, hi;
  pair_values(x, lo, hi);
  return max3(lo, hi, hi);
}

// Max of the 32 values of two MFMA accumulators: a v_max3 tree of depth 4
// (16 instructions).
__device__ __forceinline__ float max32(const f32x16& x, const f32x16& y) {
  float m[11];
#pragma unroll
  for (int i = 0; i < 5; ++i) {
    m[i] = max3(x[3 * i], x[3 * i + 1], x[3 * i + 2]);
    m[5 + i] = max3(y[3 * i], y[3 * i + 1], y[3 * i + 2]);
  }
  m[10] = max3(x[15], y[15], m[9]);
  const float a = max3(m[0], m[1], m[2]);
  const float b = max3(m[3], m[4], m[5]);
  const float c = max3(m[6], m[7], m[8]);
  return max3(a, b, max3(c, m[10], m[10]));
}

__device__ __forceinline__ float pair_sum(float x) {
  float lo, hi;
  pair_values(x, lo, hi);
  return lo + hi;
}

// Hardware dispatches workgroup b to XCD b % 8.  Map the dispatch order to a
// logical order in which XCD x owns the contiguous logical range
// [start_x, start_x + count_x), so the blocks that share a head's K/V run on
// the same L2.  Bijective for any total.
__device__ __forceinline__ int xcd_remap(int b, int total) {
  const int per = (total + kNumXcd - 1) / kNumXcd;
  int tall = total % kNumXcd;
  if (tall == 0) tall = kNumXcd;
  const int xcd = b % kNumXcd;
  const int local = b / kNumXcd;
  if (xcd < tall) return xcd * per + local;
  return tall * per + (xcd - tall) * (per - 1) + local;
}


// 32-bit LDS address of a pointer into __shared__ memory.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const lds_void_t*)(p);
}

// One global_load_lds_dwordx4: lane i copies 16 bytes from
// sbase + voff (voff: this lane's 32-bit byte offset) to LDS byte address
// lds_base + 16*i (lds_base is wave-uniform, passed in M0).
// Issued from inline asm without a memory clobber on purpose: with the
// builtin (or a clobber) the compiler cannot tell which LDS bytes the
// in-flight DMA writes and puts a full vmcnt(0) wait in front of later LDS
// reads of the *other* buffer, serialising the prefetch.  Ordering is kept
// explicitly instead: the asm is volatile (never moved across the barrier or
// the s_waitcnt, which are side-effecting too), and each tile ends with
// s_waitcnt vmcnt(0) followed by a workgroup barrier before any wave reads
// the freshly written buffer; a buffer is refilled only after the barrier
// that ends the tile which last read it.  m0 (the LDS destination) is set
// inside the asm and declared clobbered; the compiler does not preserve a
// reserved register around inline asm, so nothing else in these kernels may
// use m0 (tests/test_kernel_resources.py checks the emitted assembly).
__device__ __forceinline__ void dma_16b(uint32_t voff, const char* sbase, uint32_t lds_base) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(voff), "s"(sbase), "s"(lds_base)
               : "m0");
}

// Two ds_read_b64_tr_b16 (the gfx950 transposing LDS read) at LDS byte
// addresses addr+OFF0 and addr+OFF1, concatenated into one 8 x 16-bit MFMA
// operand.  Within each 16-lane group, lane i receives element (i & 3) of
// the 4 x 16-bit words addressed by lanes 4e + (i >> 2), e = 0..3.
template <int OFF0, int OFF1>
__device__ __forceinline__ i16x8 ds_read_tr_pair(uint32_t addr) {
  static_assert(OFF0 >= 0 && OFF1 < 65536, "ds offset field is 16 bits");
  typedef __attribute__((address_space(3))) const char lds_char_t;
  lds_char_t* p = (lds_char_t*)(uintptr_t)addr;
  const i16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(p + OFF0));
  const i16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(p + OFF1));
  return i16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

}  // namespace dev
}  // namespace fa
