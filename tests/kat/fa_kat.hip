// Known-answer-test kernels for the gfx950 instructions the forward kernel is
// built on.  Test infrastructure (tests/test_gpu_kat.py), not product code.
//
// Re-derives the reference's MMA fragment KATs (tests/unit/ptx/
// test_mma_fragment.cu:184-213 constant case, :76-121 non-integer patterns;
// tests/unit/loadstore/test_copy_srm.cu:1247-1298 PV pattern) for
// v_mfma_f32_32x32x16_{f16,bf16} with the operand layouts the forward kernel
// assumes: A lane l holds row l%32, k = 8*(l/32)..+7; B lane l holds column
// l%32, same k; D lane l, register i holds column l%32, row
// 8*(i/4) + 4*(l/32) + i%4.  Also records the lane map of ds_read_b64_tr_b16.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __attribute__((address_space(3))) i16x4 lds_i16x4_t;

__global__ void kat_mfma_kernel(const i16x8* a, const i16x8* b, const float* c, float* d, int bf16) {
  const int l = threadIdx.x;
  f32x16 acc;
  for (int i = 0; i < 16; ++i) acc[i] = c[l * 16 + i];
  if (bf16)
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a[l]),
                                                 __builtin_bit_cast(bf16x8, b[l]), acc, 0, 0, 0);
  else
    acc = __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a[l]),
                                                __builtin_bit_cast(f16x8, b[l]), acc, 0, 0, 0);
  for (int i = 0; i < 16; ++i) d[l * 16 + i] = acc[i];
}

__global__ void kat_tr_kernel(short* out) {
  __shared__ short lds[1024];
  const int l = threadIdx.x;
  for (int i = l; i < 1024; i += 64) lds[i] = (short)i;
  __syncthreads();
  const i16x4 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4_t*)(lds + 4 * l));
  for (int e = 0; e < 4; ++e) out[l * 4 + e] = r[e];
}

static int check(hipError_t e) { return e == hipSuccess ? 0 : (int)e; }

// a_bits: 32x16 row-major (16-bit patterns), b_bits: 16x32 row-major,
// c: 32x32 row-major initial accumulator, d: 32x32 result.  Returns 0 or a
// HIP error code.
extern "C" int kat_mfma_32x32x16(int bf16, const uint16_t* a_bits, const uint16_t* b_bits,
                                 const float* c, float* d) {
  uint16_t ha[64 * 8], hb[64 * 8];
  float hc[64 * 16], hd[64 * 16];
  for (int l = 0; l < 64; ++l)
    for (int i = 0; i < 8; ++i) {
      const int rc = l % 32, k = 8 * (l / 32) + i;
      ha[l * 8 + i] = a_bits[rc * 16 + k];
      hb[l * 8 + i] = b_bits[k * 32 + rc];
    }
  for (int l = 0; l < 64; ++l)
    for (int i = 0; i < 16; ++i) {
      const int col = l % 32, row = 8 * (i / 4) + 4 * (l / 32) + (i % 4);
      hc[l * 16 + i] = c[row * 32 + col];
    }
  void *da = 0, *db = 0, *dc = 0, *dd = 0;
  int rc = check(hipMalloc(&da, sizeof(ha)));
  if (!rc) rc = check(hipMalloc(&db, sizeof(hb)));
  if (!rc) rc = check(hipMalloc(&dc, sizeof(hc)));
  if (!rc) rc = check(hipMalloc(&dd, sizeof(hd)));
  if (!rc) rc = check(hipMemcpy(da, ha, sizeof(ha), hipMemcpyHostToDevice));
  if (!rc) rc = check(hipMemcpy(db, hb, sizeof(hb), hipMemcpyHostToDevice));
  if (!rc) rc = check(hipMemcpy(dc, hc, sizeof(hc), hipMemcpyHostToDevice));
  if (!rc) {
    hipLaunchKernelGGL(kat_mfma_kernel, dim3(1), dim3(64), 0, 0, (const i16x8*)da,
                       (const i16x8*)db, (const float*)dc, (float*)dd, bf16);
    rc = check(hipGetLastError());
  }
  if (!rc) rc = check(hipDeviceSynchronize());
  if (!rc) rc = check(hipMemcpy(hd, dd, sizeof(hd), hipMemcpyDeviceToHost));
  if (!rc)
    for (int l = 0; l < 64; ++l)
      for (int i = 0; i < 16; ++i) {
        const int col = l % 32, row = 8 * (i / 4) + 4 * (l / 32) + (i % 4);
        d[row * 32 + col] = hd[l * 16 + i];
      }
  if (da) (void)hipFree(da);
  if (db) (void)hipFree(db);
  if (dc) (void)hipFree(dc);
  if (dd) (void)hipFree(dd);
  return rc;
}

// out[64*4]: what each lane receives from ds_read_b64_tr_b16 when lane j
// addresses the four 16-bit words 4j..4j+3 of an LDS array holding 0..1023.
extern "C" int kat_ds_read_tr16(int16_t* out) {
  void* d = 0;
  int rc = check(hipMalloc(&d, 64 * 4 * 2));
  if (!rc) {
    hipLaunchKernelGGL(kat_tr_kernel, dim3(1), dim3(64), 0, 0, (short*)d);
    rc = check(hipGetLastError());
  }
  if (!rc) rc = check(hipDeviceSynchronize());
  if (!rc) rc = check(hipMemcpy(out, d, 64 * 4 * 2, hipMemcpyDeviceToHost));
  if (d) (void)hipFree(d);
  return rc;
}
