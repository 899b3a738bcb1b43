// fa_mfma_probe — sustained v_mfma_f32_32x32x16_f16 throughput on this GPU.
//
// Usage: fa_mfma_probe [--ms T] [--rounds R]
//
// Cross-check of the MFMA peak the benchmark divides by (256 CUs x clock x
// 4096 dense fp16 flop/clk/CU): every wave runs nothing but independent
// 32x32x16 MFMAs (four accumulator chains, sixteen distinct A/B operand pairs
// per loop body), and the flop rate is timed with HIP events.
//
// Each launch is sized to last about T ms (default 50) and is run once
// untimed first: the chip is power-limited, and its clock falls during the
// first milliseconds of a dense load.  Two operand sets are run, because the
// sustained clock also depends on how many operand bits toggle: all-ones (few
// toggles) and N(0, 1) fp16 (the benchmark inputs).  Each set runs with one
// and with two waves per SIMD (one workgroup of 4 or 8 waves per CU, kept to
// one per CU by its LDS reservation), and at each of the 8 code alignments
// of its loop within a 32-byte instruction-fetch block.  The power manager
// carries state from one launch to the next, so the configurations are
// interleaved over R rounds (default 3).
//
// The reference has no counterpart (its peak is a name-substring table,
// benchmark/cpp/include/perf_metrics.cuh:78-120); this is the "MFMA-only
// microbenchmark" cross-check of the measurement plan.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

namespace {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kOperands = 8;        // distinct A and B operands per lane
constexpr int kOperandHalves = 8;   // halves per operand per lane
constexpr int kLdsBytes = 96 * 1024;  // > 160 KiB / 2: one workgroup per CU

#define CHECK(x)                                                                  \
  do {                                                                            \
    const hipError_t e_ = (x);                                                    \
    if (e_ != hipSuccess) {                                                       \
      std::fprintf(stderr, "%s:%d: %s\n", __FILE__, __LINE__, hipGetErrorString(e_)); \
      std::exit(1);                                                               \
    }                                                                             \
  } while (0)

// PAD s_nop instructions (4 bytes each) in front of the loop: they shift the
// loop's code alignment within a 32-byte instruction-fetch block.
template <int PAD>
__device__ __forceinline__ void pad_code() {
  if constexpr (PAD > 0) {
    asm volatile("s_nop 0");
    pad_code<PAD - 1>();
  }
}

// ops: kOperands * 2 operands x 64 lanes x 8 halves, read once per thread.
// out: one float per thread (keeps the accumulators live).
template <int PAD>
__global__ void __launch_bounds__(512) mfma_loop(const _Float16* __restrict__ ops, float* out,
                                                 int iters) {
  __shared__ char lds_reserve[kLdsBytes];
  const int lane = threadIdx.x & 63;
  f16x8 a[kOperands], b[kOperands];
#pragma unroll
  for (int i = 0; i < kOperands; ++i) {
    a[i] = *reinterpret_cast<const f16x8*>(ops + ((2 * i) * 64 + lane) * kOperandHalves);
    b[i] = *reinterpret_cast<const f16x8*>(ops + ((2 * i + 1) * 64 + lane) * kOperandHalves);
  }
  f32x16 acc[4];
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[c][i] = 0.0f;
  __builtin_amdgcn_s_waitcnt(0);
  pad_code<PAD>();
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < 16; ++j)
      acc[j & 3] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[j & 7], b[(j + (j >> 3)) & 7],
                                                          acc[j & 3], 0, 0, 0);
  }
  float s = 0.0f;
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int i = 0; i < 16; ++i) s += acc[c][i];
  if (iters < 0) {  // never taken; keeps the LDS reservation in the kernel
    lds_reserve[threadIdx.x] = (char)s;
    __syncthreads();
    s += lds_reserve[threadIdx.x ^ 1];
  }
  out[blockIdx.x * blockDim.x + threadIdx.x] = s;
}

uint64_t splitmix(uint64_t& st) {
  uint64_t z = (st += 0x9e3779b97f4a7c15ull);
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

std::vector<_Float16> make_ops(bool random) {
  std::vector<_Float16> h(size_t(kOperands) * 2 * 64 * kOperandHalves);
  uint64_t st = 1234;
  for (size_t i = 0; i < h.size(); ++i) {
    if (!random) {
      h[i] = (_Float16)1.0f;
      continue;
    }
    // Box-Muller from two uniforms in (0, 1].
    const double u1 = ((splitmix(st) >> 11) + 1.0) / 9007199254740992.0;
    const double u2 = ((splitmix(st) >> 11) + 1.0) / 9007199254740992.0;
    h[i] = (_Float16)(float)(std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2));
  }
  return h;
}

struct Timing {
  double tflops;
  float ms;
};

typedef void (*LoopKernel)(const _Float16*, float*, int);
template <int P>
void fill_kernels(LoopKernel* k) {
  if constexpr (P < 8) {
    k[P] = mfma_loop<P>;
    fill_kernels<P + 1>(k);
  }
}

float time_launch(LoopKernel kern, int cus, int threads, const _Float16* d_ops, float* d_out,
                  int iters, hipEvent_t e0, hipEvent_t e1) {
  CHECK(hipEventRecord(e0, 0));
  hipLaunchKernelGGL(kern, dim3(cus), dim3(threads), 0, 0, d_ops, d_out, iters);
  CHECK(hipGetLastError());
  CHECK(hipEventRecord(e1, 0));
  CHECK(hipEventSynchronize(e1));
  float ms = 0.0f;
  CHECK(hipEventElapsedTime(&ms, e0, e1));
  return ms;
}

Timing run(LoopKernel kern, int cus, int waves_per_simd, bool random, float target_ms,
           int repeats) {
  const std::vector<_Float16> h = make_ops(random);
  _Float16* d_ops = nullptr;
  float* d_out = nullptr;
  const int threads = 256 * waves_per_simd;
  CHECK(hipMalloc(&d_ops, h.size() * sizeof(_Float16)));
  CHECK(hipMalloc(&d_out, size_t(cus) * threads * sizeof(float)));
  CHECK(hipMemcpy(d_ops, h.data(), h.size() * sizeof(_Float16), hipMemcpyHostToDevice));
  hipEvent_t e0, e1;
  CHECK(hipEventCreate(&e0));
  CHECK(hipEventCreate(&e1));
  // Size the launch (twice: the clock settles during the first one), run it
  // once untimed, then time it `repeats` times.
  int iters = 1000;
  for (int pass = 0; pass < 2; ++pass) {
    const float probe_ms = time_launch(kern, cus, threads, d_ops, d_out, iters, e0, e1);
    const double scaled = iters * (double)target_ms / (probe_ms > 1e-3f ? probe_ms : 1e-3f);
    iters = scaled < 1000.0 ? 1000 : scaled > 2e7 ? 20000000 : (int)scaled;
  }
  (void)time_launch(kern, cus, threads, d_ops, d_out, iters, e0, e1);
  std::vector<float> ms(repeats);
  for (int r = 0; r < repeats; ++r)
    ms[r] = time_launch(kern, cus, threads, d_ops, d_out, iters, e0, e1);
  std::sort(ms.begin(), ms.end());
  CHECK(hipEventDestroy(e0));
  CHECK(hipEventDestroy(e1));
  CHECK(hipFree(d_ops));
  CHECK(hipFree(d_out));
  const float med = ms[repeats / 2];
  const double flops = double(cus) * threads / 64 * double(iters) * 16 * 32 * 32 * 16 * 2;
  return {flops / (med * 1e-3) / 1e12, med};
}

}  // namespace

int main(int argc, char** argv) {
  float target_ms = 50.0f;
  int rounds = 3;
  for (int i = 1; i < argc; ++i) {
    const std::string a = argv[i];
    if ((a == "--ms" || a == "--rounds") && i + 1 < argc) {
      const double v = std::atof(argv[++i]);
      if (!(v >= 1.0 && v <= 2000.0)) {
        std::fprintf(stderr, "%s must be in [1, 2000]\n", a.c_str());
        return 2;
      }
      if (a == "--ms") target_ms = (float)v;
      else rounds = (int)v;
    } else {
      std::fprintf(stderr, "usage: %s [--ms T] [--rounds R]\n", argv[0]);
      return 2;
    }
  }
  hipDeviceProp_t prop;
  CHECK(hipGetDeviceProperties(&prop, 0));
  const int cus = prop.multiProcessorCount;
  const double peak = double(cus) * (prop.clockRate * 1e3) * 4096 / 1e12;
  std::printf("device %s, %d CUs, %.0f MHz: computed dense fp16 MFMA peak %.1f TFLOP/s\n",
              prop.gcnArchName, cus, prop.clockRate / 1e3, peak);
  // The power manager's state carries over between launches, so the four
  // configurations are interleaved over `rounds` rounds.  Each configuration
  // runs its loop at all 8 code alignments (0..28 bytes mod 32): with two
  // waves per SIMD streaming MFMAs, some alignments leave the matrix core
  // idle a third of the time.  Reported: the best alignment's median over the
  // rounds, and the range over alignments.
  LoopKernel kernels[8];
  fill_kernels<0>(kernels);
  std::vector<double> tf[4][8];
  for (int round = 0; round < rounds; ++round)
    for (int cfg = 0; cfg < 4; ++cfg)
      for (int pad = 0; pad < 8; ++pad)
        tf[cfg][pad].push_back(
            run(kernels[pad], cus, 1 + (cfg & 1), cfg >= 2, target_ms, 1).tflops);
  std::printf("%-8s %-11s %12s %8s %26s\n", "operands", "waves/SIMD", "TFLOP/s", "of peak",
              "alignments: worst-best");
  for (int cfg = 0; cfg < 4; ++cfg) {
    double best = 0.0, worst = 1e30;
    for (int pad = 0; pad < 8; ++pad) {
      std::vector<double> v = tf[cfg][pad];
      std::sort(v.begin(), v.end());
      const double med = v[v.size() / 2];
      best = std::max(best, med);
      worst = std::min(worst, med);
    }
    std::printf("%-8s %-11d %12.1f %7.1f%% %13.1f-%-9.1f\n", cfg >= 2 ? "N(0,1)" : "ones",
                1 + (cfg & 1), best, 100.0 * best / peak, worst, best);
  }
  return 0;
}
