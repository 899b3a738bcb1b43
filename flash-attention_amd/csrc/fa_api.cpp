// C ABI of the MI355X FlashAttention-2 forward library (declared in
// include/fa_mi355x.h).
//
// Host-side replacement of the reference's launch layer
// (python/flash_attention_runtime/_ext.cu:19-158): argument validation,
// kernel dispatch on the caller's stream, event timing, and the device query
// of utils/get_gpu_hardware_param.cu:1-26.  Validation is pure host code so
// every rejection branch is testable without a GPU.  The reference kernel
// silently returns on unsupported arguments (src/forward/forward_v6_mma.cuh:
// 330-339); here every unsupported argument is a status code and nothing is
// launched.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>

#include "fa_fwd_kernel.h"
#include "fa_mi355x.h"

namespace {

thread_local char g_last_error[512] = "";

fa_status fail(fa_status s, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
fa_status fail(fa_status s, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return s;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

constexpr int64_t kMaxSeqStride = int64_t(1) << 24;

// Checks one tensor's strides.  The kernels read rows with 16-byte vector
// loads, so every row start must be 16-byte aligned: the base pointer and all
// three strides (in 2-byte elements) must be multiples of 8 elements.  The
// byte offset of the last row of a head must also fit the kernels' 64-bit
// address arithmetic with a 32-bit row index.
fa_status check_strides(const char* name, const void* ptr, const int64_t st[3], int64_t seq_len,
                        int64_t head_dim) {
  for (int i = 0; i < 3; ++i) {
    if (st[i] < 0)
      return fail(FA_ERR_STRIDE, "%s stride[%d] = %lld is negative", name, i, (long long)st[i]);
    if (st[i] % 8 != 0)
      return fail(FA_ERR_STRIDE,
                  "%s stride[%d] = %lld is not a multiple of 8 elements (16-byte rows required)",
                  name, i, (long long)st[i]);
  }
  if (st[2] < head_dim && seq_len > 1)
    return fail(FA_ERR_STRIDE, "%s seq stride %lld is smaller than head_dim %lld (rows overlap)",
                name, (long long)st[2], (long long)head_dim);
  // K/V tiles are staged with 32-bit byte offsets from the tile's first row
  // (up to 63 rows of 2*stride bytes), which bounds the seq stride.
  if (st[2] > kMaxSeqStride)
    return fail(FA_ERR_UNSUPPORTED, "%s seq stride %lld exceeds %lld elements", name,
                (long long)st[2], (long long)kMaxSeqStride);
  if (!aligned16(ptr)) return fail(FA_ERR_STRIDE, "%s pointer is not 16-byte aligned", name);
  return FA_OK;
}

void to_kernel_args(const fa_fwd_params* p, fa::KernelArgs* a) {
  a->q = p->q;
  a->k = p->k;
  a->v = p->v;
  a->o = p->o;
  a->lse = p->lse;
  a->q_stride_b = p->q_stride[0];
  a->q_stride_h = p->q_stride[1];
  a->q_stride_s = p->q_stride[2];
  a->k_stride_b = p->k_stride[0];
  a->k_stride_h = p->k_stride[1];
  a->k_stride_s = p->k_stride[2];
  a->v_stride_b = p->v_stride[0];
  a->v_stride_h = p->v_stride[1];
  a->v_stride_s = p->v_stride[2];
  a->o_stride_b = p->o_stride[0];
  a->o_stride_h = p->o_stride[1];
  a->o_stride_s = p->o_stride[2];
  a->batch = p->batch;
  a->heads = p->heads;
  a->seq_len = p->seq_len;
  a->head_dim = p->head_dim;
  a->causal = p->causal;
  a->bf16 = p->dtype == FA_DTYPE_BF16;
  a->n_qblocks = 0;
  a->scale = p->softmax_scale;
  // c = scale * log2(e) (reference: src/config/config.cuh:84, forward_v6_mma.cuh:375)
  a->scale_log2 = p->softmax_scale * 1.4426950408889634f;
  a->ws_o = nullptr;
  a->ws_ml = nullptr;
  a->split.n_items = 0;
  a->split.n_slots = 0;
  a->split.n_merge = 0;
  a->split.xcd_heads = 0;
  a->split.pair = 0;
  a->split.head_group = 0;
}

// Compute units of the calling thread's current device (queried once per
// device; the split plan depends on it).
constexpr int kMaxDevices = 64;
std::atomic<int> g_device_cus[kMaxDevices];

fa_status current_compute_units(int* cus) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(FA_ERR_HIP, "hipGetDevice failed: %s", hipGetErrorString(e));
  if (dev >= 0 && dev < kMaxDevices) {
    const int cached = g_device_cus[dev].load(std::memory_order_relaxed);
    if (cached > 0) {
      *cus = cached;
      return FA_OK;
    }
  }
  e = hipDeviceGetAttribute(cus, hipDeviceAttributeMultiprocessorCount, dev);
  if (e != hipSuccess)
    return fail(FA_ERR_HIP, "device query failed: %s", hipGetErrorString(e));
  if (dev >= 0 && dev < kMaxDevices) g_device_cus[dev].store(*cus, std::memory_order_relaxed);
  return FA_OK;
}

// Validates p and launches it with the work plan for the current device:
// split over the workspace when the plan asks for one and a workspace is
// given (workspace == NULL: never split, the plain fa_fwd path), else
// possibly an XCD placement table (no workspace, same arithmetic).
fa_status launch(const fa_fwd_params* p, void* workspace, uint64_t workspace_bytes,
                 void* stream) {
  const fa_status s = fa_fwd_validate(p);
  if (s != FA_OK) return s;
  fa::KernelArgs a;
  to_kernel_args(p, &a);
  {
    int cus = 0;
    const fa_status st = current_compute_units(&cus);
    if (st != FA_OK) return st;
    const size_t need = fa::plan_split(a, cus, workspace != nullptr, &a.split);
    if (need > 0) {
      if (workspace_bytes < need)
        return fail(FA_ERR_ARG, "workspace of %llu bytes is smaller than the %llu bytes needed",
                    (unsigned long long)workspace_bytes, (unsigned long long)need);
      if (!aligned16(workspace))
        return fail(FA_ERR_STRIDE, "workspace pointer is not 16-byte aligned");
      const size_t o_bytes = (size_t)p->batch * p->heads * a.split.n_slots *
                             fa::block_rows(a) * p->head_dim * 4;
      a.ws_o = static_cast<float*>(workspace);
      a.ws_ml = reinterpret_cast<float*>(static_cast<char*>(workspace) + o_bytes);
    }
  }
  const hipError_t e = fa::launch_fwd(a, static_cast<hipStream_t>(stream));
  if (e != hipSuccess)
    return fail(FA_ERR_HIP, "kernel launch failed: %s", hipGetErrorString(e));
  return FA_OK;
}

// launch() bracketed by two HIP events on `stream`.
fa_status launch_timed(const fa_fwd_params* p, void* workspace, uint64_t workspace_bytes,
                       void* stream, float* ms) {
  if (ms == nullptr) return fail(FA_ERR_NULL, "ms is NULL");
  *ms = 0.0f;
  const fa_status s = fa_fwd_validate(p);
  if (s != FA_OK) return s;
  hipStream_t st = static_cast<hipStream_t>(stream);
  hipEvent_t start = nullptr, stop = nullptr;
  hipError_t e = hipEventCreate(&start);
  if (e == hipSuccess) e = hipEventCreate(&stop);
  if (e == hipSuccess) e = hipEventRecord(start, st);
  fa_status out = FA_OK;
  if (e == hipSuccess) {
    out = launch(p, workspace, workspace_bytes, stream);
    if (out == FA_OK) {
      e = hipEventRecord(stop, st);
      if (e == hipSuccess) e = hipEventSynchronize(stop);
      if (e == hipSuccess) e = hipEventElapsedTime(ms, start, stop);
    }
  }
  if (start) (void)hipEventDestroy(start);
  if (stop) (void)hipEventDestroy(stop);
  if (out != FA_OK) return out;
  if (e != hipSuccess) return fail(FA_ERR_HIP, "event timing failed: %s", hipGetErrorString(e));
  return FA_OK;
}

}  // namespace

extern "C" {

const char* fa_status_str(fa_status s) {
  switch (s) {
    case FA_OK: return "ok";
    case FA_ERR_NULL: return "null pointer";
    case FA_ERR_DTYPE: return "unsupported dtype (expected fp16 or bf16)";
    case FA_ERR_SHAPE: return "invalid shape (batch, heads and seq_len must be >= 1)";
    case FA_ERR_HEADDIM: return "unsupported head_dim (expected 64 or 128)";
    case FA_ERR_STRIDE: return "unsupported stride or alignment";
    case FA_ERR_UNSUPPORTED: return "problem size beyond the kernel's index range";
    case FA_ERR_HIP: return "HIP runtime error";
    case FA_ERR_ARG: return "invalid argument";
  }
  return "unknown status";
}

const char* fa_last_error(void) { return g_last_error; }

const char* fa_version(void) { return "fa_mi355x 0.1.0 gfx950"; }

fa_status fa_fwd_validate(const fa_fwd_params* p) {
  g_last_error[0] = '\0';
  if (p == nullptr) return fail(FA_ERR_NULL, "params is NULL");
  if (p->q == nullptr) return fail(FA_ERR_NULL, "q is NULL");
  if (p->k == nullptr) return fail(FA_ERR_NULL, "k is NULL");
  if (p->v == nullptr) return fail(FA_ERR_NULL, "v is NULL");
  if (p->o == nullptr) return fail(FA_ERR_NULL, "o is NULL");
  if (p->dtype != FA_DTYPE_F16 && p->dtype != FA_DTYPE_BF16)
    return fail(FA_ERR_DTYPE, "dtype %d is not fp16 (0) or bf16 (1)", (int)p->dtype);
  if (p->batch < 1 || p->heads < 1 || p->seq_len < 1)
    return fail(FA_ERR_SHAPE, "batch=%d heads=%d seq_len=%d must all be >= 1", (int)p->batch,
                (int)p->heads, (int)p->seq_len);
  if (p->head_dim != 64 && p->head_dim != 128)
    return fail(FA_ERR_HEADDIM, "Only head_dim 64 and 128 are supported (got %d)",
                (int)p->head_dim);
  if (p->causal != 0 && p->causal != 1)
    return fail(FA_ERR_ARG, "causal must be 0 or 1 (got %d)", (int)p->causal);
  // The exponent is computed as exp2(s*c - m*c) with m the running max of the
  // raw scores; that identity needs c > 0 (reference online_softmax.cuh:13-19).
  if (!std::isfinite(p->softmax_scale) || !(p->softmax_scale > 0.0f))
    return fail(FA_ERR_ARG, "softmax_scale must be finite and > 0 (got %g)",
                (double)p->softmax_scale);
  fa_status s;
  if ((s = check_strides("q", p->q, p->q_stride, p->seq_len, p->head_dim)) != FA_OK) return s;
  if ((s = check_strides("k", p->k, p->k_stride, p->seq_len, p->head_dim)) != FA_OK) return s;
  if ((s = check_strides("v", p->v, p->v_stride, p->seq_len, p->head_dim)) != FA_OK) return s;
  if ((s = check_strides("o", p->o, p->o_stride, p->seq_len, p->head_dim)) != FA_OK) return s;
  if (p->lse != nullptr && (reinterpret_cast<uintptr_t>(p->lse) & 3u) != 0)
    return fail(FA_ERR_STRIDE, "lse pointer is not 4-byte aligned");
  // Grid = batch * heads * ceil(seq_len / 128) workgroups in one dimension.
  const int64_t blocks = (int64_t)p->batch * p->heads * (((int64_t)p->seq_len + 127) / 128);
  if (blocks > 0x7fffffffLL)
    return fail(FA_ERR_UNSUPPORTED, "batch*heads*ceil(seq_len/128) = %lld exceeds 2^31-1",
                (long long)blocks);
  return FA_OK;
}

fa_status fa_fwd(const fa_fwd_params* p, void* stream) {
  return launch(p, nullptr, 0, stream);
}

fa_status fa_fwd_timed(const fa_fwd_params* p, void* stream, float* ms) {
  return launch_timed(p, nullptr, 0, stream, ms);
}

fa_status fa_fwd_plan(const fa_fwd_params* p, int32_t compute_units, fa_fwd_plan_t* out) {
  if (out == nullptr) return fail(FA_ERR_NULL, "out is NULL");
  std::memset(out, 0, sizeof(*out));
  const fa_status s = fa_fwd_validate(p);
  if (s != FA_OK) return s;
  if (compute_units < 1)
    return fail(FA_ERR_ARG, "compute_units must be >= 1 (got %d)", (int)compute_units);
  fa::KernelArgs a;
  to_kernel_args(p, &a);
  out->workspace_bytes = fa::plan_split(a, compute_units, true, &a.split);
  out->block_rows = fa::block_rows(a);
  out->n_items = a.split.n_items;
  out->n_slots = a.split.n_slots;
  out->n_merge = a.split.n_merge;
  out->xcd_heads = a.split.xcd_heads;
  out->key_halves = a.split.pair ? 2 : 1;
  out->head_group = a.split.head_group;
  for (int i = 0; i < a.split.n_items; ++i) {
    const uint32_t info = a.split.item[i];
    const int qb = (int)(info & 0xffffu), c = (int)((info >> 16) & 0xffu), nch = (int)(info >> 24);
    // The kernel's split of the q-tile's key tiles [0, T) (fa_fwd_kernel).
    const int kv = p->causal ? std::min(p->seq_len, (qb + 1) * out->block_rows) : p->seq_len;
    const int T = (kv + 63) / 64;
    out->q_tile[i] = qb;
    out->n_chunks[i] = nch;
    out->tile_begin[i] = (int32_t)((int64_t)c * T / nch);
    out->tile_end[i] = (int32_t)((int64_t)(c + 1) * T / nch);
    const bool table = a.split.xcd_heads > 0;
    out->slot[i] = nch > 1 ? a.split.slot[i] + c : -1;  // table items are never chunked
    out->head[i] = table ? a.split.slot[i] : -1;
  }
  return FA_OK;
}

fa_status fa_fwd_workspace_size(const fa_fwd_params* p, uint64_t* bytes) {
  if (bytes == nullptr) return fail(FA_ERR_NULL, "bytes is NULL");
  *bytes = 0;
  const fa_status s = fa_fwd_validate(p);
  if (s != FA_OK) return s;
  int cus = 0;
  const fa_status st = current_compute_units(&cus);
  if (st != FA_OK) return st;
  fa::KernelArgs a;
  to_kernel_args(p, &a);
  *bytes = fa::plan_split(a, cus, true, &a.split);
  return FA_OK;
}

fa_status fa_fwd_ws(const fa_fwd_params* p, void* workspace, uint64_t workspace_bytes,
                    void* stream) {
  if (workspace == nullptr && workspace_bytes != 0)
    return fail(FA_ERR_NULL, "workspace is NULL but workspace_bytes = %llu",
                (unsigned long long)workspace_bytes);
  if (workspace == nullptr) {
    // Allowed only when the problem needs no workspace.
    uint64_t need = 0;
    const fa_status s = fa_fwd_workspace_size(p, &need);
    if (s != FA_OK) return s;
    if (need > 0)
      return fail(FA_ERR_NULL, "workspace is NULL but %llu bytes are needed",
                  (unsigned long long)need);
  }
  return launch(p, workspace, workspace_bytes, stream);
}

fa_status fa_fwd_ws_timed(const fa_fwd_params* p, void* workspace, uint64_t workspace_bytes,
                          void* stream, float* ms) {
  if (workspace == nullptr && workspace_bytes != 0) {
    if (ms != nullptr) *ms = 0.0f;
    return fail(FA_ERR_NULL, "workspace is NULL but workspace_bytes = %llu",
                (unsigned long long)workspace_bytes);
  }
  if (workspace == nullptr) {
    uint64_t need = 0;
    const fa_status s = fa_fwd_workspace_size(p, &need);
    if (s != FA_OK) return s;
    if (need > 0) {
      if (ms != nullptr) *ms = 0.0f;
      return fail(FA_ERR_NULL, "workspace is NULL but %llu bytes are needed",
                  (unsigned long long)need);
    }
  }
  return launch_timed(p, workspace, workspace_bytes, stream, ms);
}

fa_status fa_fwd_scratch(const fa_fwd_params* p, void* stream) {
  static_assert(fa::kScratchBytes == FA_SCRATCH_BYTES, "header and library disagree");
  uint64_t need = 0;
  const fa_status s = fa_fwd_workspace_size(p, &need);
  if (s != FA_OK) return s;
  if (need == 0) return launch(p, nullptr, 0, stream);
  if (need > fa::kScratchBytes)
    return fail(FA_ERR_UNSUPPORTED,
                "the split-KV plan needs %llu bytes of workspace; the static scratch holds %llu "
                "(use fa_fwd_ws with a caller workspace, or fa_fwd)",
                (unsigned long long)need, (unsigned long long)fa::kScratchBytes);
  void* ws = nullptr;
  const hipError_t e = fa::scratch_buffer(&ws);
  if (e != hipSuccess)
    return fail(FA_ERR_HIP, "scratch lookup failed: %s", hipGetErrorString(e));
  return launch(p, ws, fa::kScratchBytes, stream);
}

fa_status fa_device_info(int device, fa_device_info_t* out) {
  if (out == nullptr) return fail(FA_ERR_NULL, "out is NULL");
  std::memset(out, 0, sizeof(*out));
  hipDeviceProp_t prop;
  const hipError_t e = hipGetDeviceProperties(&prop, device);
  if (e != hipSuccess)
    return fail(FA_ERR_HIP, "hipGetDeviceProperties(%d) failed: %s", device, hipGetErrorString(e));
  std::snprintf(out->arch, sizeof(out->arch), "%s", prop.gcnArchName);
  // Some driver installs report an empty marketing name; fall back to the ISA.
  std::snprintf(out->name, sizeof(out->name), "%s", prop.name[0] ? prop.name : prop.gcnArchName);
  out->compute_units = prop.multiProcessorCount;
  out->clock_khz = prop.clockRate;
  out->lds_per_cu_bytes = (int64_t)prop.maxSharedMemoryPerMultiProcessor;
  out->l2_bytes = prop.l2CacheSize;
  out->memory_bus_width_bits = prop.memoryBusWidth;
  out->memory_clock_khz = prop.memoryClockRate;
  out->global_mem_bytes = (int64_t)prop.totalGlobalMem;
  out->lds_per_block_bytes = (int64_t)prop.sharedMemPerBlock;
  out->regs_per_block = prop.regsPerBlock;
  out->regs_per_cu = prop.regsPerMultiprocessor;
  out->max_threads_per_cu = prop.maxThreadsPerMultiProcessor;
  out->max_threads_per_block = prop.maxThreadsPerBlock;
  out->wavefront_size = prop.warpSize;
  out->arch_major = prop.major;
  out->arch_minor = prop.minor;
  // CDNA4: 2048 dense fp16/bf16 FMA = 4096 flop per clock per CU.
  out->fp16_dense_peak_tflops = (double)prop.multiProcessorCount * prop.clockRate * 1e3 * 4096.0 / 1e12;
  // The DDR formula below does not hold for HBM3E's data rate; for gfx950
  // (MI355X) use the published 8 TB/s, as the reference keys its peak table
  // on the device (perf_metrics.cuh:78-120).
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) == 0)
    out->hbm_peak_gbps = 8000.0;
  else
    out->hbm_peak_gbps = 2.0 * prop.memoryClockRate * 1e3 * (prop.memoryBusWidth / 8.0) / 1e9;
  return FA_OK;
}

}  // extern "C"
