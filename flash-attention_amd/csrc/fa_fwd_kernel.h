// Internal interface between the C ABI (fa_api.cpp) and the HIP kernels.
// Mirrors the reference's kernel argument block ForwardKernelArgs
// (src/config/config.cuh:20-45) with 64-bit strides, dtype, LSE and the
// precomputed exponent scale.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fa {

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
};

// Launches the forward kernel for args (validated by the caller) on stream.
hipError_t launch_fwd(const KernelArgs& args, hipStream_t stream);

}  // namespace fa
