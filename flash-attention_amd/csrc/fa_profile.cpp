// fa_profile — command-line benchmark of the forward through the C ABI.
//
// Replaces the reference's C++ benchmark executable
// (benchmark/cpp/benchmark_v6.cu:201-348, with its shape table
// benchmark/cpp/include/test_configs.h:14-17 and report
// benchmark/cpp/include/perf_metrics.cuh:33-75,124-163):
//
//   fa_profile [config|BxHxNxD] [--mode benchmark|rocprof] [--warmup-iters N]
//              [--benchmark-iters N] [--dtype fp16|bf16] [--causal] [--seed S]
//
// `--mode rocprof` (the reference's `--mode ncu`) defaults to 0 warmup and 1
// timed launch, for running under `rocprofv3 --kernel-trace` or `--pmc`.
// Inputs are uniform in [0, 1) as the reference's rand()/RAND_MAX fill, from a
// seeded splitmix64 stream, rounded to the input type on the host.
//
// Per case it prints a report and one line
//   CSV,B,H,N,d,time_ms,gflops,compute_efficiency,memory_gb,bandwidth_gb_s,
//       bandwidth_utilization,throughput_tokens_ms,throughput_tokens_sec
// in the reference's column order (perf_metrics.cuh:70-75), with the
// reference's FLOP count B*H*(4N^2 d + 6N^2) (perf_metrics.cuh:140) so the
// line can be compared with the reference's logs, and additionally
// "TFLOPS(4BHN^2D)" — the metric this library is measured on, halved for
// causal.  Everything device-side goes through include/fa_mi355x.h.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "fa_mi355x.h"

namespace {

struct Shape {
  std::string name;
  int B, H, N, D;
};

// The reference's default table plus the configs this library is measured on.
const Shape kShapes[] = {
    {"tiny", 2, 4, 512, 64},          {"small", 4, 8, 1024, 128},
    {"medium", 8, 16, 2048, 128},     {"large", 8, 16, 4096, 128},
    {"c2", 4, 16, 1024, 64},          {"c3", 4, 32, 4096, 128},
    {"c4", 2, 32, 8192, 128},         {"c5", 1, 16, 16384, 128},
    {"c5r", 1, 16, 3000, 128},
};

#define HIP_OK(call)                                                                   \
  do {                                                                                 \
    hipError_t e_ = (call);                                                            \
    if (e_ != hipSuccess) {                                                            \
      fprintf(stderr, "HIP error %s at %s:%d\n", hipGetErrorString(e_), __FILE__, __LINE__); \
      exit(1);                                                                         \
    }                                                                                  \
  } while (0)

uint64_t splitmix64(uint64_t& s) {
  uint64_t z = (s += 0x9E3779B97F4A7C15ull);
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}

// float -> IEEE binary16 bits, round to nearest even (inputs here are finite
// and in [0, 1)).
uint16_t to_f16(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  const uint32_t sign = (x >> 16) & 0x8000u;
  x &= 0x7fffffffu;
  if (x < 0x33000001u) return (uint16_t)sign;  // rounds to +-0
  if (x < 0x38800000u) {                       // subnormal half
    const int e = (int)(x >> 23);
    const uint32_t m = (x & 0x7fffffu) | 0x800000u;
    const int shift = 126 - e;  // 14 - (e - 127) - 1 + 24 - 23
    uint32_t h = m >> shift;
    const uint32_t rem = m & ((1u << shift) - 1), half = 1u << (shift - 1);
    if (rem > half || (rem == half && (h & 1u))) ++h;
    return (uint16_t)(sign | h);
  }
  uint32_t h = ((x - 0x38000000u) >> 13);
  const uint32_t rem = x & 0x1fffu;
  if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h;
  return (uint16_t)(sign | h);
}

uint16_t to_bf16(float f) {
  uint32_t x;
  std::memcpy(&x, &f, 4);
  const uint32_t lsb = (x >> 16) & 1u;
  return (uint16_t)((x + 0x7fffu + lsb) >> 16);
}

struct Result {
  float ms;
  double ref_flops, gflops, eff, mem_gb, bw, bw_util, tok_ms, tok_s, tflops_metric;
};

Result run_case(const Shape& s, int dtype, int causal, int warmup, int iters, uint64_t seed,
                const fa_device_info_t& info) {
  const size_t n = (size_t)s.B * s.H * s.N * s.D;
  std::vector<uint16_t> host(n);
  void* buf[4];
  for (int t = 0; t < 4; ++t) HIP_OK(hipMalloc(&buf[t], n * 2));
  uint64_t st = seed;
  for (int t = 0; t < 3; ++t) {
    for (size_t i = 0; i < n; ++i) {
      const float u = (float)(splitmix64(st) >> 40) * (1.0f / 16777216.0f);
      host[i] = dtype == FA_DTYPE_BF16 ? to_bf16(u) : to_f16(u);
    }
    HIP_OK(hipMemcpy(buf[t], host.data(), n * 2, hipMemcpyHostToDevice));
  }
  fa_fwd_params p;
  std::memset(&p, 0, sizeof p);
  p.q = buf[0];
  p.k = buf[1];
  p.v = buf[2];
  p.o = buf[3];
  p.lse = nullptr;
  const int64_t stride[3] = {(int64_t)s.H * s.N * s.D, (int64_t)s.N * s.D, s.D};
  for (int i = 0; i < 3; ++i)
    p.q_stride[i] = p.k_stride[i] = p.v_stride[i] = p.o_stride[i] = stride[i];
  p.batch = s.B;
  p.heads = s.H;
  p.seq_len = s.N;
  p.head_dim = s.D;
  p.softmax_scale = 1.0f / std::sqrt((float)s.D);
  p.causal = causal;
  p.dtype = dtype;

  fa_status rc = fa_fwd_validate(&p);
  if (rc != FA_OK) {
    fprintf(stderr, "%s: %s: %s\n", s.name.c_str(), fa_status_str(rc), fa_last_error());
    exit(1);
  }
  for (int i = 0; i < warmup; ++i) {
    if ((rc = fa_fwd(&p, nullptr)) != FA_OK) {
      fprintf(stderr, "fa_fwd: %s\n", fa_last_error());
      exit(1);
    }
  }
  HIP_OK(hipDeviceSynchronize());
  hipEvent_t a, b;
  HIP_OK(hipEventCreate(&a));
  HIP_OK(hipEventCreate(&b));
  HIP_OK(hipEventRecord(a, nullptr));
  for (int i = 0; i < iters; ++i) {
    if ((rc = fa_fwd(&p, nullptr)) != FA_OK) {
      fprintf(stderr, "fa_fwd: %s\n", fa_last_error());
      exit(1);
    }
  }
  HIP_OK(hipEventRecord(b, nullptr));
  HIP_OK(hipEventSynchronize(b));
  float total = 0.0f;
  HIP_OK(hipEventElapsedTime(&total, a, b));
  HIP_OK(hipEventDestroy(a));
  HIP_OK(hipEventDestroy(b));
  for (int t = 0; t < 4; ++t) HIP_OK(hipFree(buf[t]));

  Result r;
  r.ms = total / iters;
  const double B = s.B, H = s.H, N = s.N, D = s.D;
  r.ref_flops = B * H * (4.0 * N * N * D + 6.0 * N * N);
  r.gflops = r.ref_flops / (r.ms * 1e-3) / 1e9;
  r.eff = 100.0 * r.gflops / (info.fp16_dense_peak_tflops * 1e3);
  r.mem_gb = 4.0 * B * H * N * D * 2.0 / (1024.0 * 1024.0 * 1024.0);
  r.bw = r.mem_gb / (r.ms * 1e-3);
  r.bw_util = info.hbm_peak_gbps > 0 ? 100.0 * r.bw / info.hbm_peak_gbps : 0.0;
  r.tok_ms = B * H * N / r.ms;
  r.tok_s = r.tok_ms * 1e3;
  r.tflops_metric = 4.0 * B * H * N * N * D / (causal ? 2.0 : 1.0) / (r.ms * 1e-3) / 1e12;
  return r;
}

bool parse_shape(const char* text, Shape& out) {
  int b, h, n, d;
  char tail;
  if (std::sscanf(text, "%dx%dx%dx%d%c", &b, &h, &n, &d, &tail) != 4) return false;
  if (b <= 0 || h <= 0 || n <= 0 || d <= 0) return false;
  out = {"custom", b, h, n, d};
  return true;
}

void usage(const char* argv0) {
  printf("Usage: %s [config|BxHxNxD] [--mode benchmark|rocprof] [--warmup-iters N]\n"
         "          [--benchmark-iters N] [--dtype fp16|bf16] [--causal] [--seed S]\n"
         "configs:", argv0);
  for (const Shape& s : kShapes) printf(" %s", s.name.c_str());
  printf("\n  mode=benchmark default: warmup=10, benchmark=100\n"
         "  mode=rocprof default: warmup=0, benchmark=1\n");
}

}  // namespace

int main(int argc, char** argv) {
  bool rocprof = false, causal = false;
  int warmup = -1, iters = -1, dtype = FA_DTYPE_F16;
  uint64_t seed = 1234;
  const char* token = nullptr;
  for (int i = 1; i < argc; ++i) {
    const std::string a = argv[i];
    auto value = [&](const char* what) -> const char* {
      if (i + 1 >= argc) {
        fprintf(stderr, "%s requires a value\n", what);
        exit(1);
      }
      return argv[++i];
    };
    if (a == "-h" || a == "--help") {
      usage(argv[0]);
      return 0;
    } else if (a == "--mode") {
      const std::string m = value("--mode");
      if (m == "benchmark") rocprof = false;
      else if (m == "rocprof" || m == "ncu") rocprof = true;
      else {
        fprintf(stderr, "Invalid --mode: %s (expected benchmark|rocprof)\n", m.c_str());
        return 1;
      }
    } else if (a == "--warmup-iters") {
      warmup = std::max(0, std::atoi(value("--warmup-iters")));
    } else if (a == "--benchmark-iters") {
      iters = std::max(1, std::atoi(value("--benchmark-iters")));
    } else if (a == "--dtype") {
      const std::string d = value("--dtype");
      if (d == "fp16") dtype = FA_DTYPE_F16;
      else if (d == "bf16") dtype = FA_DTYPE_BF16;
      else {
        fprintf(stderr, "Invalid --dtype: %s (expected fp16|bf16)\n", d.c_str());
        return 1;
      }
    } else if (a == "--causal") {
      causal = true;
    } else if (a == "--seed") {
      seed = std::strtoull(value("--seed"), nullptr, 10);
    } else if (a.rfind("--", 0) == 0) {
      fprintf(stderr, "Unknown option: %s\n", a.c_str());
      return 1;
    } else if (token != nullptr) {
      fprintf(stderr, "Unexpected extra positional argument: %s\n", a.c_str());
      return 1;
    } else {
      token = argv[i];
    }
  }
  if (warmup < 0) warmup = rocprof ? 0 : 10;
  if (iters < 0) iters = rocprof ? 1 : 100;

  std::vector<Shape> cases;
  Shape custom;
  if (token == nullptr) {
    for (const Shape& s : kShapes)
      if (s.name == "tiny" || s.name == "small" || s.name == "medium" || s.name == "large")
        cases.push_back(s);
  } else if (parse_shape(token, custom)) {
    cases.push_back(custom);
  } else {
    for (const Shape& s : kShapes)
      if (s.name == token) cases.push_back(s);
    if (cases.empty()) {
      fprintf(stderr, "Unknown config: %s\n", token);
      usage(argv[0]);
      return 1;
    }
  }

  fa_device_info_t info;
  if (fa_device_info(0, &info) != FA_OK) {
    fprintf(stderr, "fa_device_info: %s\n", fa_last_error());
    return 1;
  }
  printf("GPU 0: %s (%s), %d CUs, %.0f MHz, dense fp16/bf16 MFMA peak %.1f TFLOPS, "
         "HBM %.0f GB/s\n", info.name, info.arch, info.compute_units, info.clock_khz / 1e3,
         info.fp16_dense_peak_tflops, info.hbm_peak_gbps);
  printf("%s, mode=%s, warmup=%d, iters=%d, dtype=%s, causal=%d\n", fa_version(),
         rocprof ? "rocprof" : "benchmark", warmup, iters,
         dtype == FA_DTYPE_BF16 ? "bf16" : "fp16", (int)causal);

  std::vector<std::pair<Shape, Result>> results;
  for (const Shape& s : cases) {
    const Result r = run_case(s, dtype, causal ? 1 : 0, warmup, iters, seed, info);
    printf("\n--- %s: B=%d H=%d N=%d d=%d ---\n", s.name.c_str(), s.B, s.H, s.N, s.D);
    printf("  Time: %.4f ms\n", r.ms);
    printf("  TFLOPS(4BHN^2D%s): %.2f\n", causal ? "/2" : "", r.tflops_metric);
    printf("  Reference FLOPs B*H*(4N^2d+6N^2): %.3e -> %.2f GFLOPS (%.1f%% of peak)\n",
           r.ref_flops, r.gflops, r.eff);
    printf("  Memory: %.3f GB, %.2f GB/s (%.1f%% of peak)\n", r.mem_gb, r.bw, r.bw_util);
    printf("  Throughput: %.2f K tokens/ms, %.2f M tokens/s\n", r.tok_ms / 1e3, r.tok_s / 1e6);
    printf("CSV,%d,%d,%d,%d,%.3f,%.2f,%.1f,%.2f,%.2f,%.1f,%.2f,%.2f\n", s.B, s.H, s.N, s.D, r.ms,
           r.gflops, r.eff, r.mem_gb, r.bw, r.bw_util, r.tok_ms, r.tok_s);
    results.emplace_back(s, r);
  }
  printf("\n%-10s %5s %5s %8s %5s %10s %12s %10s\n", "Config", "B", "H", "N", "d", "Time(ms)",
         "GFLOPS", "TFLOPS*");
  for (const auto& [s, r] : results)
    printf("%-10s %5d %5d %8d %5d %10.4f %12.2f %10.2f\n", s.name.c_str(), s.B, s.H, s.N, s.D,
           r.ms, r.gflops, r.tflops_metric);
  printf("(* 4*B*H*N^2*D%s per launch)\n", causal ? ", halved for causal" : "");
  return 0;
}
