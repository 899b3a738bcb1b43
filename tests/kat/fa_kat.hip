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

#include "fa_device_ops.h"

using namespace fa::dev;

__global__ void kat_mfma_kernel(const i16x8* a, const i16x8* b, const float* c, float* d, int bf16) {
  const int l = threadIdx.x;
  f32x16 acc;
  for (int i = 0; i < 16; ++i) acc[i] = c[l * 16 + i];
  acc = bf16 ? ElemOps<true>::mfma(a[l], b[l], acc) : ElemOps<false>::mfma(a[l], b[l], acc);
  for (int i = 0; i < 16; ++i) d[l * 16 + i] = acc[i];
}

// ds_read_tr_pair<0, 512>: lane j addresses words 4j..4j+3 (first read) and
// 256+4j..256+4j+3 (second read) of an LDS array holding 0..1023.
__global__ void kat_tr_kernel(short* out) {
  __shared__ short lds[1024];
  const int l = threadIdx.x;
  for (int i = l; i < 1024; i += 64) lds[i] = (short)i;
  __syncthreads();
  const i16x8 r = ds_read_tr_pair<0, 512>(lds_addr(lds + 4 * l));
  for (int e = 0; e < 8; ++e) out[l * 8 + e] = r[e];
}

__global__ void kat_pack_kernel(const float* in, uint32_t* out, float* dot, int bf16) {
  const int l = threadIdx.x;
  const uint32_t w = bf16 ? pack2<true>(in[2 * l], in[2 * l + 1]) : pack2<false>(in[2 * l], in[2 * l + 1]);
  out[l] = w;
  dot[l] = bf16 ? dot2_acc<true>(w, 0.25f) : dot2_acc<false>(w, 0.25f);
}

__global__ void kat_pair_kernel(const float* in, float* mx, float* sm) {
  const int l = threadIdx.x;
  mx[l] = pair_max(in[l]);
  sm[l] = pair_sum(in[l]);
}

// dma_16b: lane i fetches 16 bytes from src + 16*((i * 7) % 64) into LDS
// bytes [16*i, 16*i + 16) of the second 1 KiB of a 2 KiB buffer.
__global__ void kat_dma_kernel(const char* src, int* out) {
  __shared__ __attribute__((aligned(1024))) int buf[512];
  const int l = threadIdx.x;
  for (int i = l; i < 512; i += 64) buf[i] = -1;
  __syncthreads();
  const uint32_t base = __builtin_amdgcn_readfirstlane(lds_addr(buf)) + 1024;
  dma_16b((uint32_t)(16 * ((l * 7) % 64)), src, base);
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  for (int i = l; i < 512; i += 64) out[i] = buf[i];
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

// out[64*8]: the two transposed reads of ds_read_tr_pair<0, 512> per lane.
extern "C" int kat_ds_read_tr16(int16_t* out) {
  void* d = 0;
  int rc = check(hipMalloc(&d, 64 * 8 * 2));
  if (!rc) {
    hipLaunchKernelGGL(kat_tr_kernel, dim3(1), dim3(64), 0, 0, (short*)d);
    rc = check(hipGetLastError());
  }
  if (!rc) rc = check(hipDeviceSynchronize());
  if (!rc) rc = check(hipMemcpy(out, d, 64 * 8 * 2, hipMemcpyDeviceToHost));
  if (d) (void)hipFree(d);
  return rc;
}

// in[128] floats -> out[64] packed pairs (pack2) and dot[64] = 0.25 + sum of
// the pair (dot2_acc).
extern "C" int kat_pack2(int bf16, const float* in, uint32_t* out, float* dot) {
  void *di = 0, *dout = 0, *ddot = 0;
  int rc = check(hipMalloc(&di, 128 * 4));
  if (!rc) rc = check(hipMalloc(&dout, 64 * 4));
  if (!rc) rc = check(hipMalloc(&ddot, 64 * 4));
  if (!rc) rc = check(hipMemcpy(di, in, 128 * 4, hipMemcpyHostToDevice));
  if (!rc) {
    hipLaunchKernelGGL(kat_pack_kernel, dim3(1), dim3(64), 0, 0, (const float*)di,
                       (uint32_t*)dout, (float*)ddot, bf16);
    rc = check(hipGetLastError());
  }
  if (!rc) rc = check(hipDeviceSynchronize());
  if (!rc) rc = check(hipMemcpy(out, dout, 64 * 4, hipMemcpyDeviceToHost));
  if (!rc) rc = check(hipMemcpy(dot, ddot, 64 * 4, hipMemcpyDeviceToHost));
  if (di) (void)hipFree(di);
  if (dout) (void)hipFree(dout);
  if (ddot) (void)hipFree(ddot);
  return rc;
}

// in[64] -> pair_max / pair_sum of lanes l and l^32.
extern "C" int kat_pair(const float* in, float* mx, float* sm) {
  void *di = 0, *dm = 0, *ds = 0;
  int rc = check(hipMalloc(&di, 64 * 4));
  if (!rc) rc = check(hipMalloc(&dm, 64 * 4));
  if (!rc) rc = check(hipMalloc(&ds, 64 * 4));
  if (!rc) rc = check(hipMemcpy(di, in, 64 * 4, hipMemcpyHostToDevice));
  if (!rc) {
    hipLaunchKernelGGL(kat_pair_kernel, dim3(1), dim3(64), 0, 0, (const float*)di, (float*)dm,
                       (float*)ds);
    rc = check(hipGetLastError());
  }
  if (!rc) rc = check(hipDeviceSynchronize());
  if (!rc) rc = check(hipMemcpy(mx, dm, 64 * 4, hipMemcpyDeviceToHost));
  if (!rc) rc = check(hipMemcpy(sm, ds, 64 * 4, hipMemcpyDeviceToHost));
  if (di) (void)hipFree(di);
  if (dm) (void)hipFree(dm);
  if (ds) (void)hipFree(ds);
  return rc;
}

// src: 1 KiB of int32 0..255 -> out[512]: the 2 KiB LDS buffer after one DMA.
extern "C" int kat_dma(int* out) {
  int host[256];
  for (int i = 0; i < 256; ++i) host[i] = i;
  void *dsrc = 0, *dout = 0;
  int rc = check(hipMalloc(&dsrc, 1024));
  if (!rc) rc = check(hipMalloc(&dout, 2048));
  if (!rc) rc = check(hipMemcpy(dsrc, host, 1024, hipMemcpyHostToDevice));
  if (!rc) {
    hipLaunchKernelGGL(kat_dma_kernel, dim3(1), dim3(64), 0, 0, (const char*)dsrc, (int*)dout);
    rc = check(hipGetLastError());
  }
  if (!rc) rc = check(hipDeviceSynchronize());
  if (!rc) rc = check(hipMemcpy(out, dout, 2048, hipMemcpyDeviceToHost));
  if (dsrc) (void)hipFree(dsrc);
  if (dout) (void)hipFree(dout);
  return rc;
}

__global__ void kat_xcd_kernel(int total, int* out) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b < total) out[b] = fa::dev::xcd_remap(b, total);
}

// out[b] = xcd_remap(b, total) for every dispatch index b < total.
extern "C" int kat_xcd_remap(int total, int* out) {
  if (total < 1) return -1;
  void* d = 0;
  int rc = check(hipMalloc(&d, (size_t)total * 4));
  if (!rc) {
    hipLaunchKernelGGL(kat_xcd_kernel, dim3((total + 255) / 256), dim3(256), 0, 0, total, (int*)d);
    rc = check(hipGetLastError());
  }
  if (!rc) rc = check(hipDeviceSynchronize());
  if (!rc) rc = check(hipMemcpy(out, d, (size_t)total * 4, hipMemcpyDeviceToHost));
  if (d) (void)hipFree(d);
  return rc;
}

// row_sum_mfma / row_sum_of_lane over two P chunks: lane l holds 8 fp16 or
// bf16 values (bits in p_bits[(c*64 + l)*8 ..]) of chunk c; out[l] receives
// the sum over both chunks of row l % 32 (lanes l%32 and l%32 + 32), the
// first chunk's sums scaled by row_sum_scale with the factor of row r held
// in f[r] and f[r + 32] (as the kernel holds per-row values).
template <bool BF16>
__global__ void kat_row_sum_kernel(const i16x8* p, const float* f, float* out) {
  const int l = threadIdx.x;
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
  const i16x8 sel = row_sum_selector<BF16>(l);
  acc = row_sum_mfma<BF16>(sel, p[l], acc);
  acc = row_sum_scale(acc, f[l], l);
  acc = row_sum_mfma<BF16>(sel, p[64 + l], acc);
  out[l] = row_sum_of_lane(acc, l);
}

extern "C" int kat_row_sum(const uint16_t* p_bits, const float* f, int bf16, float* out) {
  void *dp = 0, *df = 0, *dout = 0;
  int rc = check(hipMalloc(&dp, 2 * 64 * 8 * 2));
  if (!rc) rc = check(hipMalloc(&df, 64 * 4));
  if (!rc) rc = check(hipMalloc(&dout, 64 * 4));
  if (!rc) rc = check(hipMemcpy(dp, p_bits, 2 * 64 * 8 * 2, hipMemcpyHostToDevice));
  if (!rc) rc = check(hipMemcpy(df, f, 64 * 4, hipMemcpyHostToDevice));
  if (!rc) {
    if (bf16)
      hipLaunchKernelGGL(kat_row_sum_kernel<true>, dim3(1), dim3(64), 0, 0, (const i16x8*)dp,
                         (const float*)df, (float*)dout);
    else
      hipLaunchKernelGGL(kat_row_sum_kernel<false>, dim3(1), dim3(64), 0, 0, (const i16x8*)dp,
                         (const float*)df, (float*)dout);
    rc = check(hipGetLastError());
  }
  if (!rc) rc = check(hipDeviceSynchronize());
  if (!rc) rc = check(hipMemcpy(out, dout, 64 * 4, hipMemcpyDeviceToHost));
  if (dp) (void)hipFree(dp);
  if (df) (void)hipFree(df);
  if (dout) (void)hipFree(dout);
  return rc;
}
