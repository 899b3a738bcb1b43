/*
 * fa_mi355x.h — C ABI of the MI355X (gfx950) FlashAttention-2 forward library.
 *
 * This is the drop-in boundary for the reference's forward path.  Every entry
 * point takes plain pointers and sizes; no torch or HIP types appear in the
 * signatures (a HIP stream is passed as `void*`, NULL meaning the null stream).
 *
 * Reference interfaces replaced (paths under the reference repository):
 *   - fa_fwd          <- launch_fp16 + the kernel launch
 *                        python/flash_attention_runtime/_ext.cu:59-122,
 *                        and the kernel argument block ForwardKernelArgs
 *                        src/config/config.cuh:20-45
 *   - fa_fwd_validate <- validate_inputs / check_cuda_tensor
 *                        python/flash_attention_runtime/_ext.cu:19-57
 *   - fa_fwd_timed    <- fa_forward(..., benchmark=true) event timing
 *                        python/flash_attention_runtime/_ext.cu:124-158
 *   - fa_device_info  <- utils/get_gpu_hardware_param.cu:1-26 and the peak
 *                        table infer_device_peak_specs
 *                        benchmark/cpp/include/perf_metrics.cuh:78-120
 *   - fa_fwd_ws, fa_fwd_ws_timed, fa_fwd_workspace_size, fa_fwd_plan:
 *                        no counterpart in the reference (its kernel has one
 *                        workgroup per q-tile); the workspace variants of
 *                        fa_fwd / fa_fwd_timed add split-KV for problems
 *                        whose grid would leave most CUs idle behind a few
 *                        long q-tiles (short causal sequences, few heads).
 *   - fa_fwd_scratch:    no counterpart in the reference; fa_fwd_ws for
 *                        callers that cannot allocate (see its comment).
 *
 * Semantics (all entry points):
 *   O[b,h,i,:] = sum_j softmax_j(scale * Q[b,h,i,:].K[b,h,j,:] + mask_ij) V[b,h,j,:]
 *   LSE[b,h,i] = ln sum_j exp(scale * Q[b,h,i,:].K[b,h,j,:] + mask_ij)   (natural log)
 *   mask_ij = -inf when causal and j > i (top-left aligned), else 0.
 * Tensors are [batch, heads, seq_len, head_dim] with unit stride along
 * head_dim; the batch/head/seq strides are free (so BNHD views work without a
 * copy) up to a seq stride of 2^24 elements (FA_ERR_UNSUPPORTED beyond).
 * O has the input dtype; LSE is fp32 [batch, heads, seq_len], contiguous,
 * and optional.
 *
 * Ownership: all pointers are borrowed; the library allocates no device memory
 * (the split-KV partials live in a workspace the caller provides, or, for
 * fa_fwd_scratch, in a static array of FA_SCRATCH_BYTES per device).
 * Threading: re-entrant; the only mutable global state is a thread-local error
 * string, a per-device cache of the CU count (written once, atomically), the
 * per-device address of the scratch array (looked up once, under a lock) and
 * that array's contents (fa_fwd_scratch only).
 * Streams: fa_fwd is asynchronous on `stream`; unlike the reference
 * kernel, an unsupported argument never turns into a silent device no-op —
 * it is rejected on the host with a status code before anything is launched.
 */
#ifndef FA_MI355X_H
#define FA_MI355X_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
  FA_OK = 0,
  FA_ERR_NULL = 1,        /* a required pointer is NULL                          */
  FA_ERR_DTYPE = 2,       /* dtype is not FA_DTYPE_F16 / FA_DTYPE_BF16           */
  FA_ERR_SHAPE = 3,       /* batch, heads or seq_len < 1                         */
  FA_ERR_HEADDIM = 4,     /* head_dim not in {64, 128}                           */
  FA_ERR_STRIDE = 5,      /* negative / misaligned stride or pointer             */
  FA_ERR_UNSUPPORTED = 6, /* shape beyond the kernels' index range               */
  FA_ERR_HIP = 7,         /* a HIP runtime call failed (see fa_last_error)       */
  FA_ERR_ARG = 8          /* softmax_scale not finite and > 0, causal not 0/1    */
} fa_status;

typedef enum { FA_DTYPE_F16 = 0, FA_DTYPE_BF16 = 1 } fa_dtype;

/* Kernel argument block.  Mirrors ForwardKernelArgs (src/config/config.cuh:20-45)
 * with 64-bit strides, a dtype tag, the causal flag and an optional LSE output.
 * Strides are in elements: [0] batch, [1] head, [2] seq.  head_dim stride is 1. */
typedef struct {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  float* lse; /* may be NULL: then no logsumexp is written */
  int64_t q_stride[3];
  int64_t k_stride[3];
  int64_t v_stride[3];
  int64_t o_stride[3];
  int32_t batch;
  int32_t heads;
  int32_t seq_len;
  int32_t head_dim;
  float softmax_scale; /* the reference passes 1/sqrt(head_dim) (_ext.cu:93) */
  int32_t causal;      /* 0 or 1 */
  int32_t dtype;       /* fa_dtype */
} fa_fwd_params;

/* Device description (replaces utils/get_gpu_hardware_param.cu:1-26). */
typedef struct {
  char name[256];
  char arch[64];
  int32_t compute_units;
  int32_t clock_khz;
  int64_t lds_per_cu_bytes;
  int64_t l2_bytes;
  int32_t memory_bus_width_bits;
  int32_t memory_clock_khz;
  /* compute_units x clock x 4096 dense fp16/bf16 MFMA flop per clock per CU */
  double fp16_dense_peak_tflops;
  /* published 8000 GB/s for gfx950 (MI355X); 2 x bus width x memory clock
   * (DDR) for other devices */
  double hbm_peak_gbps;
  /* the remaining fields of utils/get_gpu_hardware_param.cu:11-24 */
  int64_t global_mem_bytes;      /* totalGlobalMem */
  int64_t lds_per_block_bytes;   /* sharedMemPerBlock */
  int32_t regs_per_block;        /* regsPerBlock */
  int32_t regs_per_cu;           /* regsPerMultiprocessor */
  int32_t max_threads_per_cu;    /* maxThreadsPerMultiProcessor */
  int32_t max_threads_per_block; /* maxThreadsPerBlock */
  int32_t wavefront_size;        /* warpSize (64 on CDNA) */
  int32_t arch_major;            /* major (gfx9xx: 9) */
  int32_t arch_minor;            /* minor */
  int32_t reserved;
} fa_device_info_t;

/* Work plan of a problem (diagnostic; filled by fa_fwd_plan): split-KV, an XCD
 * placement table, pair mode, or none. */
#define FA_PLAN_MAX_ITEMS 128
typedef struct {
  int32_t block_rows;       /* query rows per workgroup (q-tile height) of the kernel */
  int32_t n_items;          /* workgroups per (batch, head); 0: the problem runs unsplit */
  int32_t n_slots;          /* partial-result slots per (batch, head) in the workspace */
  int32_t n_merge;          /* q-tiles with more than one chunk (merged by a second kernel) */
  int32_t xcd_heads;        /* > 0: XCD placement table (no split) over this many heads per XCD */
  int32_t key_halves;       /* 2: pair mode (8 waves per q-tile, each half on alternate key
                               tiles, one workgroup per q-tile, no items); 1 otherwise */
  int32_t head_group;       /* > 0: causal grid without items, B*H a multiple of 8: each XCD
                               runs its heads in groups of this many, the q-tiles of a group
                               interleaved longest first; 0 otherwise */
  int32_t reserved;         /* 0 */
  uint64_t workspace_bytes; /* bytes fa_fwd_ws needs (0 when unsplit) */
  /* Split-KV (xcd_heads == 0): work item i (dispatch order, longest first)
   * of every (batch, head) is q-tile q_tile[i], key tiles (64 keys each)
   * [tile_begin[i], tile_end[i]) of its n_chunks[i] chunks, partial slot
   * slot[i] (-1 for a q-tile of one chunk, stored directly).
   * XCD placement table (xcd_heads > 0): the i-th workgroup dispatched to
   * each XCD runs q-tile q_tile[i] of head head[i] among that XCD's
   * xcd_heads heads, all its key tiles.  fa_fwd uses the same table. */
  int32_t q_tile[FA_PLAN_MAX_ITEMS];
  int32_t tile_begin[FA_PLAN_MAX_ITEMS];
  int32_t tile_end[FA_PLAN_MAX_ITEMS];
  int32_t n_chunks[FA_PLAN_MAX_ITEMS];
  int32_t slot[FA_PLAN_MAX_ITEMS];
  int32_t head[FA_PLAN_MAX_ITEMS];
} fa_fwd_plan_t;

/* Host-only argument check; touches no GPU.  Returns FA_OK or the first
 * failing rule (see fa_status).  Replaces _ext.cu:19-57. */
fa_status fa_fwd_validate(const fa_fwd_params* p);

/* Validate, then launch the forward kernel asynchronously on `stream`
 * (a hipStream_t; NULL = null stream).  Replaces _ext.cu:59-122. */
fa_status fa_fwd(const fa_fwd_params* p, void* stream);

/* fa_fwd bracketed by two HIP events on `stream`; blocks until the kernel has
 * finished and writes its elapsed time in milliseconds to *ms.
 * Replaces the benchmark=true branch of fa_forward (_ext.cu:136-155). */
fa_status fa_fwd_timed(const fa_fwd_params* p, void* stream, float* ms);

/* Workspace bytes fa_fwd_ws needs for *p on the calling thread's current
 * device (0: the problem runs unsplit and fa_fwd_ws equals fa_fwd).
 * Queries the device's CU count; launches nothing. */
fa_status fa_fwd_workspace_size(const fa_fwd_params* p, uint64_t* bytes);

/* fa_fwd with a device workspace of `workspace_bytes` bytes (16-byte
 * aligned, contents undefined on entry, overwritten): long key ranges may be
 * split across workgroups whose fp32 partials go to the workspace and are
 * merged by a second kernel on `stream`.  The result equals fa_fwd's within
 * fp32 rounding of the merge (not bit for bit).  FA_ERR_ARG if workspace_bytes
 * is below fa_fwd_workspace_size; workspace may be NULL only when that size
 * is 0.  Calls that share a workspace must be ordered (same stream). */
fa_status fa_fwd_ws(const fa_fwd_params* p, void* workspace, uint64_t workspace_bytes,
                    void* stream);

/* fa_fwd_ws bracketed by two HIP events on `stream`, as fa_fwd_timed. */
fa_status fa_fwd_ws_timed(const fa_fwd_params* p, void* workspace, uint64_t workspace_bytes,
                          void* stream, float* ms);

/* Bytes of the library's static split-KV scratch (one array per device). */
#define FA_SCRATCH_BYTES (32ull << 20)

/* fa_fwd_ws with the library's own static device scratch array as the
 * workspace: allocates nothing (no hipMalloc, no allocating library call).
 * No counterpart in the reference; it is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid allocation).  The array (FA_SCRATCH_BYTES per device) is part
 * of the library's device code object: it is reserved when the first launch
 * of any entry point of the library on a device loads that code object there
 * (as every HIP module's globals are), and held until the process ends; its
 * address is looked up on the first fa_fwd_scratch call per device.  A caller
 * that must see no device allocation at all from this call makes one launch of
 * the library on that device beforehand (any entry point).  A problem whose
 * split-KV plan needs more than FA_SCRATCH_BYTES is rejected with
 * FA_ERR_UNSUPPORTED and nothing is launched.  Every call on one device
 * shares that device's array, which keeps the last call's contents: calls
 * that overlap on one device (other streams, other host threads) race and
 * must be ordered by the caller.  Same results as fa_fwd_ws. */
fa_status fa_fwd_scratch(const fa_fwd_params* p, void* stream);

/* The work plan fa_fwd_ws would use for *p on a device with
 * `compute_units` CUs (split-KV, an XCD placement table, pair mode, or none).
 * Host only; touches no GPU. */
fa_status fa_fwd_plan(const fa_fwd_params* p, int32_t compute_units, fa_fwd_plan_t* out);

/* Static description of a status code. */
const char* fa_status_str(fa_status s);

/* Detail of the last failure on the calling thread ("" if none).  The string
 * belongs to the library (thread-local storage) and stays valid until the
 * same thread's next call into the library. */
const char* fa_last_error(void);

/* Query device `device`.  Returns FA_OK, FA_ERR_NULL or FA_ERR_HIP. */
fa_status fa_device_info(int device, fa_device_info_t* out);

/* Library version string, e.g. "fa_mi355x 0.1.0 gfx950". */
const char* fa_version(void);

#ifdef __cplusplus
}
#endif

#endif /* FA_MI355X_H */
