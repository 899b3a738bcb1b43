// fa_correctness — C++ correctness check of the forward through the C ABI.
//
// TEST INFRASTRUCTURE: built by tests/cpp/build_cpp.py into tests/cpp/ and
// run by tests/test_gpu_cpp_tools.py::test_cpp_correctness_executable;
// never linked into libfa_mi355x.so.  It links the library
// (include/fa_mi355x.h) and the CPU oracle (oracle/liboracle.so) as the
// checker.
//
// Replaces the reference's benchmark/cpp/correctness_v6.cu:106-217.  Case 0
// is that file's case: B=1 H=1 N=64 D=128 fp16, non-causal, inputs
// (rand()/RAND_MAX - 0.5) * 0.2 after srand(17), the CPU reference
// cpu_reference_attention (:23-72, restated as oracle_ref_online_f32) run on
// the unrounded fp32 inputs, and check_close over every element with
// atol 2e-2, rtol 8e-2 (:74-104).  The other cases go beyond the reference's
// path (ragged N, causal, bf16, head_dim 64, N(0,1) inputs) and are checked
// against the fp64 oracle on the rounded inputs at the contract bars
// (max-abs 1e-2, mean-abs 1e-3, LSE 1e-3).
//
// Exit status 0 when every case passes.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "attn_oracle.h"
#include "fa_mi355x.h"

namespace {

bool hip_ok(hipError_t e, const char* what) {
  if (e == hipSuccess) return true;
  std::printf("%s failed: %s\n", what, hipGetErrorString(e));
  return false;
}

// correctness_v6.cu:74-104: |ref - out| <= atol + rtol * |ref| element-wise.
bool check_close(const float* ref, const float* out, int64_t n, float atol, float rtol) {
  float max_diff = 0.0f;
  int64_t max_idx = 0, fails = 0;
  for (int64_t i = 0; i < n; ++i) {
    const float diff = std::fabs(ref[i] - out[i]);
    const float tol = atol + rtol * std::fabs(ref[i]);
    if (!(diff <= tol)) {
      if (fails < 10)
        std::printf("  mismatch [%lld]: ref=%.6f out=%.6f diff=%.6f tol=%.6f\n", (long long)i,
                    ref[i], out[i], diff, tol);
      ++fails;
    }
    if (diff > max_diff) {
      max_diff = diff;
      max_idx = i;
    }
  }
  std::printf("  check_close(atol %.0e, rtol %.0e): max abs diff %.3e at %lld, %lld / %lld "
              "mismatches\n", atol, rtol, max_diff, (long long)max_idx, (long long)fails,
              (long long)n);
  return fails == 0;
}

// splitmix64 -> uniform [0, 1), Box-Muller -> N(0, 1)
struct Rng {
  uint64_t s;
  double uniform() {
    uint64_t z = (s += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    z ^= z >> 31;
    return (z >> 11) * (1.0 / 9007199254740992.0);
  }
  float normal() {
    const double u1 = uniform() + 1e-300, u2 = uniform();
    return (float)(std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2));
  }
};

struct Case {
  const char* name;
  int B, H, N, D, causal, dtype;
  int reference_inputs;  // 1: correctness_v6.cu's inputs and check
};

float bits_to_float(uint16_t b, int dtype) {
  if (dtype == FA_DTYPE_BF16) {
    const uint32_t x = (uint32_t)b << 16;
    float f;
    std::memcpy(&f, &x, 4);
    return f;
  }
  _Float16 h;
  std::memcpy(&h, &b, 2);
  return (float)h;
}

bool run_case(const Case& c, unsigned seed) {
  const int64_t E = (int64_t)c.B * c.H * c.N * c.D;
  const int64_t R = (int64_t)c.B * c.H * c.N;
  const float scale = 1.0f / std::sqrt((float)c.D);
  std::printf("case %s: B=%d H=%d N=%d D=%d %s causal=%d\n", c.name, c.B, c.H, c.N, c.D,
              c.dtype == FA_DTYPE_BF16 ? "bf16" : "fp16", c.causal);
  std::vector<float> qf(E), kf(E), vf(E);
  if (c.reference_inputs) {
    srand(seed);  // correctness_v6.cu:121-129
    for (int64_t i = 0; i < E; ++i) {
      qf[i] = ((float)rand() / RAND_MAX - 0.5f) * 0.2f;
      kf[i] = ((float)rand() / RAND_MAX - 0.5f) * 0.2f;
      vf[i] = ((float)rand() / RAND_MAX - 0.5f) * 0.2f;
    }
  } else {
    Rng g{seed};
    for (int64_t i = 0; i < E; ++i) qf[i] = g.normal();
    for (int64_t i = 0; i < E; ++i) kf[i] = g.normal();
    for (int64_t i = 0; i < E; ++i) vf[i] = g.normal();
  }
  // Rounded inputs (what the GPU computes on) as bits and as floats.
  std::vector<uint16_t> qb(E), kb(E), vb(E);
  std::vector<float> qr(E), kr(E), vr(E);
  auto round = c.dtype == FA_DTYPE_BF16 ? oracle_round_bf16 : oracle_round_f16;
  round(qf.data(), qr.data(), qb.data(), E);
  round(kf.data(), kr.data(), kb.data(), E);
  round(vf.data(), vr.data(), vb.data(), E);

  void *dq = nullptr, *dk = nullptr, *dv = nullptr, *dout = nullptr;
  float* dlse = nullptr;
  bool ok = hip_ok(hipMalloc(&dq, E * 2), "hipMalloc(q)") && hip_ok(hipMalloc(&dk, E * 2), "hipMalloc(k)") &&
            hip_ok(hipMalloc(&dv, E * 2), "hipMalloc(v)") && hip_ok(hipMalloc(&dout, E * 2), "hipMalloc(o)") &&
            hip_ok(hipMalloc((void**)&dlse, R * 4), "hipMalloc(lse)");
  ok = ok && hip_ok(hipMemcpy(dq, qb.data(), E * 2, hipMemcpyHostToDevice), "copy q") &&
       hip_ok(hipMemcpy(dk, kb.data(), E * 2, hipMemcpyHostToDevice), "copy k") &&
       hip_ok(hipMemcpy(dv, vb.data(), E * 2, hipMemcpyHostToDevice), "copy v") &&
       hip_ok(hipMemset(dout, 0, E * 2), "memset o");
  std::vector<uint16_t> ob(E);
  std::vector<float> lse(R), out(E);
  if (ok) {
    fa_fwd_params p;
    std::memset(&p, 0, sizeof(p));
    p.q = dq;
    p.k = dk;
    p.v = dv;
    p.o = dout;
    p.lse = dlse;
    const int64_t st[3] = {(int64_t)c.H * c.N * c.D, (int64_t)c.N * c.D, c.D};
    for (int i = 0; i < 3; ++i) p.q_stride[i] = p.k_stride[i] = p.v_stride[i] = p.o_stride[i] = st[i];
    p.batch = c.B;
    p.heads = c.H;
    p.seq_len = c.N;
    p.head_dim = c.D;
    p.softmax_scale = scale;
    p.causal = c.causal;
    p.dtype = c.dtype;
    const fa_status s = fa_fwd(&p, nullptr);
    if (s != FA_OK) {
      std::printf("  fa_fwd failed: %s: %s\n", fa_status_str(s), fa_last_error());
      ok = false;
    }
    ok = ok && hip_ok(hipDeviceSynchronize(), "kernel");
    ok = ok && hip_ok(hipMemcpy(ob.data(), dout, E * 2, hipMemcpyDeviceToHost), "copy o") &&
         hip_ok(hipMemcpy(lse.data(), dlse, R * 4, hipMemcpyDeviceToHost), "copy lse");
  }
  hipFree(dq);
  hipFree(dk);
  hipFree(dv);
  hipFree(dout);
  hipFree(dlse);
  if (!ok) return false;
  for (int64_t i = 0; i < E; ++i) out[i] = bits_to_float(ob[i], c.dtype);

  bool pass = true;
  if (c.reference_inputs) {
    // correctness_v6.cu:132, :215: the reference runs its CPU path on the
    // unrounded fp32 inputs and compares with atol 2e-2, rtol 8e-2.
    std::vector<float> ref(E);
    if (oracle_ref_online_f32(qf.data(), kf.data(), vf.data(), ref.data(), c.B, c.H, c.N, c.D,
                              scale, c.causal, 0, R) != 0)
      return false;
    std::printf("  first 8 reference: ");
    for (int i = 0; i < 8; ++i) std::printf("%.6f ", ref[i]);
    std::printf("\n  first 8 output:    ");
    for (int i = 0; i < 8; ++i) std::printf("%.6f ", out[i]);
    std::printf("\n");
    pass = check_close(ref.data(), out.data(), E, 2e-2f, 8e-2f) && pass;
  }
  // fp64 oracle on the rounded inputs: the contract bars.
  std::vector<double> ro(E), rl(R);
  if (oracle_attn_f64(qr.data(), kr.data(), vr.data(), ro.data(), rl.data(), c.B, c.H, c.N, c.D,
                      scale, c.causal, ORACLE_MUT_NONE) != 0)
    return false;
  double mx = 0, sum = 0, lmx = 0;
  for (int64_t i = 0; i < E; ++i) {
    const double d = std::fabs((double)out[i] - ro[i]);
    mx = d > mx ? d : mx;
    sum += d;
  }
  for (int64_t i = 0; i < R; ++i) {
    const double d = std::fabs((double)lse[i] - rl[i]);
    lmx = d > lmx ? d : lmx;
  }
  const double mean = sum / (double)E;
  const bool bars = mx <= 1e-2 && mean <= 1e-3 && lmx <= 1e-3 && std::isfinite(mx);
  std::printf("  vs fp64 oracle: max_abs %.3e mean_abs %.3e lse %.3e -> %s\n", mx, mean, lmx,
              bars ? "ok" : "FAIL");
  return pass && bars;
}

}  // namespace

int main() {
  fa_device_info_t info;
  if (fa_device_info(0, &info) == FA_OK)
    std::printf("device: %s (%s), %d CUs\n", info.name, info.arch, info.compute_units);
  const Case cases[] = {
      {"reference_v6", 1, 1, 64, 128, 0, FA_DTYPE_F16, 1},
      {"single_row", 1, 2, 1, 64, 0, FA_DTYPE_F16, 0},
      {"ragged", 1, 2, 65, 128, 0, FA_DTYPE_F16, 0},
      {"ragged_causal", 2, 2, 129, 64, 1, FA_DTYPE_F16, 0},
      {"bf16_causal", 1, 3, 300, 128, 1, FA_DTYPE_BF16, 0},
      {"bf16_d64", 2, 2, 257, 64, 0, FA_DTYPE_BF16, 0},
      {"wide_rows", 1, 2, 2304, 128, 0, FA_DTYPE_F16, 0},
  };
  int failed = 0;
  unsigned seed = 17;  // correctness_v6.cu:120
  for (const Case& c : cases) {
    const bool ok = run_case(c, seed);
    std::printf("  %s\n", ok ? "PASS" : "FAIL");
    failed += ok ? 0 : 1;
    seed = seed * 1103515245u + 12345u;
  }
  std::printf("%s: %d of %zu cases failed\n", failed ? "FAILED" : "ALL PASSED", failed,
              sizeof(cases) / sizeof(cases[0]));
  return failed ? 1 : 0;
}
