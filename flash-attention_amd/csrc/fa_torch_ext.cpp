// PyTorch host binding of the MI355X FlashAttention-2 forward.
//
// Mirrors the reference's pybind extension python/flash_attention_runtime/
// _ext.cu (check_cuda_tensor / validate_inputs :19-57, launch_fp16 :59-122,
// fa_forward :124-158, PYBIND11_MODULE :162-173): same positional signature
// and result, forward(q, k, v, o=None, benchmark=False) -> (o, ms) with ms
// = 0 unless benchmark, the same validation messages where the rule is the
// same, output allocated with empty_like(q) when o is not given, launch on
// the current stream.  It adds keyword-only arguments causal, softmax_scale,
// return_lse (then the result is (o, ms, lse)) and split_kv, and accepts
// bf16, head_dim 64, any seq_len >= 1 and strided [B,H,N,D] views with unit
// head_dim stride.  With split_kv the split-KV workspace comes from torch's
// caching allocator on the current stream.
//
// All device work goes through the C ABI in include/fa_mi355x.h; this file
// holds no kernels and no HIP calls besides fetching the current stream.
#include <torch/extension.h>

#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>
#include <c10/core/DeviceGuard.h>

#include <cmath>
#include <optional>

#include "fa_mi355x.h"

namespace {

void check_device_tensor(const torch::Tensor& t, const char* name) {
  TORCH_CHECK(t.is_cuda(), name, " must be a CUDA tensor");
  TORCH_CHECK(t.dim() == 4, name, " must be a 4D tensor with shape [B, H, N, D]");
  TORCH_CHECK(t.dtype() == torch::kFloat16 || t.dtype() == torch::kBFloat16, name,
              " must be float16 or bfloat16");
  TORCH_CHECK(t.stride(3) == 1, name, " must have unit stride in the last dimension");
}

void validate_inputs(const torch::Tensor& q, const torch::Tensor& k, const torch::Tensor& v,
                     const std::optional<torch::Tensor>& o_opt) {
  check_device_tensor(q, "q");
  check_device_tensor(k, "k");
  check_device_tensor(v, "v");
  TORCH_CHECK(q.sizes() == k.sizes(), "q and k must have the same shape");
  TORCH_CHECK(q.sizes() == v.sizes(), "q and v must have the same shape");
  TORCH_CHECK(q.dtype() == k.dtype(), "q and k must have the same dtype");
  TORCH_CHECK(q.dtype() == v.dtype(), "q and v must have the same dtype");
  TORCH_CHECK(k.device() == q.device() && v.device() == q.device(),
              "q, k and v must be on the same device");
  const auto d = q.size(3);
  TORCH_CHECK(d == 64 || d == 128, "Only head_dim 64 and 128 are supported");
  if (o_opt.has_value()) {
    const auto& o = o_opt.value();
    check_device_tensor(o, "o");
    TORCH_CHECK(o.sizes() == q.sizes(), "o must have the same shape as q");
    TORCH_CHECK(o.dtype() == q.dtype(), "o must have the same dtype as q");
    TORCH_CHECK(o.device() == q.device(), "o must be on the same device as q");
  }
}

fa_fwd_params make_params(const torch::Tensor& q, const torch::Tensor& k, const torch::Tensor& v,
                          torch::Tensor& o, float* lse, bool causal, double scale) {
  fa_fwd_params p{};
  p.q = q.data_ptr();
  p.k = k.data_ptr();
  p.v = v.data_ptr();
  p.o = o.data_ptr();
  p.lse = lse;
  for (int i = 0; i < 3; ++i) {
    p.q_stride[i] = q.stride(i);
    p.k_stride[i] = k.stride(i);
    p.v_stride[i] = v.stride(i);
    p.o_stride[i] = o.stride(i);
  }
  p.batch = static_cast<int32_t>(q.size(0));
  p.heads = static_cast<int32_t>(q.size(1));
  p.seq_len = static_cast<int32_t>(q.size(2));
  p.head_dim = static_cast<int32_t>(q.size(3));
  p.softmax_scale = static_cast<float>(scale);
  p.causal = causal ? 1 : 0;
  p.dtype = q.dtype() == torch::kBFloat16 ? FA_DTYPE_BF16 : FA_DTYPE_F16;
  return p;
}

// Returns (o, ms), or (o, ms, lse) with return_lse: the reference's callers
// index and unpack the pair (python/flash_attention_runtime/__init__.py:31,37).
pybind11::tuple fa_forward(
    const torch::Tensor& q, const torch::Tensor& k, const torch::Tensor& v,
    std::optional<torch::Tensor> o_opt, bool benchmark, bool causal,
    std::optional<double> softmax_scale, bool return_lse, bool split_kv) {
  validate_inputs(q, k, v, o_opt);
  TORCH_CHECK(q.size(0) <= INT32_MAX && q.size(1) <= INT32_MAX && q.size(2) <= INT32_MAX,
              "shape does not fit 32-bit sizes");
  const c10::OptionalDeviceGuard guard(q.device());

  torch::Tensor o = o_opt.has_value() ? o_opt.value() : torch::empty_like(q);
  std::optional<torch::Tensor> lse;
  if (return_lse)
    lse = torch::empty({q.size(0), q.size(1), q.size(2)}, q.options().dtype(torch::kFloat32));

  // Reference default: softmax_scale = 1/sqrt(head_dim) (_ext.cu:93).
  const double scale =
      softmax_scale.has_value() ? softmax_scale.value() : 1.0 / std::sqrt((double)q.size(3));
  fa_fwd_params p = make_params(q, k, v, o, lse ? lse->data_ptr<float>() : nullptr, causal, scale);
  void* stream = at::hip::getCurrentHIPStreamMasqueradingAsCUDA(q.device().index()).stream();

  uint64_t ws_bytes = 0;
  if (split_kv) {
    const fa_status s = fa_fwd_workspace_size(&p, &ws_bytes);
    TORCH_CHECK(s == FA_OK, "flash attention forward failed: ", fa_status_str(s), ": ",
                fa_last_error());
  }
  torch::Tensor ws;
  if (ws_bytes > 0) ws = torch::empty({(int64_t)ws_bytes}, q.options().dtype(torch::kUInt8));
  void* wsp = ws_bytes > 0 ? ws.data_ptr() : nullptr;

  float ms = 0.0f;
  fa_status s;
  if (split_kv)
    s = benchmark ? fa_fwd_ws_timed(&p, wsp, ws_bytes, stream, &ms)
                  : fa_fwd_ws(&p, wsp, ws_bytes, stream);
  else
    s = benchmark ? fa_fwd_timed(&p, stream, &ms) : fa_fwd(&p, stream);
  TORCH_CHECK(s == FA_OK, "flash attention forward failed: ", fa_status_str(s), ": ",
              fa_last_error());
  if (return_lse) return pybind11::make_tuple(o, static_cast<double>(ms), *lse);
  return pybind11::make_tuple(o, static_cast<double>(ms));
}

pybind11::dict device_info(int device) {
  fa_device_info_t info;
  const fa_status s = fa_device_info(device, &info);
  TORCH_CHECK(s == FA_OK, "fa_device_info failed: ", fa_last_error());
  pybind11::dict d;
  d["name"] = std::string(info.name);
  d["arch"] = std::string(info.arch);
  d["compute_units"] = info.compute_units;
  d["clock_khz"] = info.clock_khz;
  d["lds_per_cu_bytes"] = info.lds_per_cu_bytes;
  d["l2_bytes"] = info.l2_bytes;
  d["memory_bus_width_bits"] = info.memory_bus_width_bits;
  d["memory_clock_khz"] = info.memory_clock_khz;
  d["fp16_dense_peak_tflops"] = info.fp16_dense_peak_tflops;
  d["hbm_peak_gbps"] = info.hbm_peak_gbps;
  d["global_mem_bytes"] = info.global_mem_bytes;
  d["lds_per_block_bytes"] = info.lds_per_block_bytes;
  d["regs_per_block"] = info.regs_per_block;
  d["regs_per_cu"] = info.regs_per_cu;
  d["max_threads_per_cu"] = info.max_threads_per_cu;
  d["max_threads_per_block"] = info.max_threads_per_block;
  d["wavefront_size"] = info.wavefront_size;
  d["arch_major"] = info.arch_major;
  d["arch_minor"] = info.arch_minor;
  return d;
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
  m.def("forward", &fa_forward, pybind11::arg("q"), pybind11::arg("k"), pybind11::arg("v"),
        pybind11::arg("o") = std::optional<torch::Tensor>{}, pybind11::arg("benchmark") = false,
        pybind11::kw_only(),
        pybind11::arg("causal") = false, pybind11::arg("softmax_scale") = std::optional<double>{},
        pybind11::arg("return_lse") = false, pybind11::arg("split_kv") = true,
        "FlashAttention-2 forward (MI355X / gfx950, HIP)");
  m.def("device_info", &device_info, pybind11::arg("device") = 0,
        "hipDeviceProp summary and dense fp16/bf16 MFMA peak");
  m.def("version", []() { return std::string(fa_version()); });
}
