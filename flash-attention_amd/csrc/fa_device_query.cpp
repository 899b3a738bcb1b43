// fa_device_query — prints the device description the library uses.
//
// Replaces the reference's utils/get_gpu_hardware_param.cu:1-26 (a
// cudaDeviceProp dump) with the hipDeviceProp fields through the C ABI's
// fa_device_info, in the same order, under AMD names (LDS for shared memory,
// CU for SM, wavefront for warp), plus the derived dense fp16/bf16 MFMA peak
// and HBM peak the benchmarks divide by.
//
//   fa_device_query [device] [--json]
#include <cstdio>
#include <cstdlib>
#include <cstring>

#include "fa_mi355x.h"

int main(int argc, char** argv) {
  int device = 0;
  bool json = false;
  for (int i = 1; i < argc; ++i) {
    if (std::strcmp(argv[i], "--json") == 0)
      json = true;
    else
      device = std::atoi(argv[i]);
  }
  fa_device_info_t d;
  const fa_status s = fa_device_info(device, &d);
  if (s != FA_OK) {
    std::fprintf(stderr, "fa_device_info failed: %s: %s\n", fa_status_str(s), fa_last_error());
    return 1;
  }
  if (json) {
    std::printf(
        "{\"name\": \"%s\", \"arch\": \"%s\", \"global_mem_mb\": %lld, \"lds_per_block_kb\": %lld, "
        "\"lds_per_cu_kb\": %lld, \"regs_per_block\": %d, \"regs_per_cu\": %d, \"l2_kb\": %lld, "
        "\"arch_major\": %d, \"arch_minor\": %d, \"compute_units\": %d, "
        "\"max_threads_per_cu\": %d, \"max_threads_per_block\": %d, \"wavefront_size\": %d, "
        "\"clock_khz\": %d, \"fp16_dense_peak_tflops\": %.1f, \"hbm_peak_gbps\": %.1f}\n",
        d.name, d.arch, (long long)(d.global_mem_bytes >> 20), (long long)(d.lds_per_block_bytes >> 10),
        (long long)(d.lds_per_cu_bytes >> 10), d.regs_per_block, d.regs_per_cu,
        (long long)(d.l2_bytes >> 10), d.arch_major, d.arch_minor, d.compute_units,
        d.max_threads_per_cu, d.max_threads_per_block, d.wavefront_size, d.clock_khz,
        d.fp16_dense_peak_tflops, d.hbm_peak_gbps);
    return 0;
  }
  std::printf("--- GPU Hardware Properties for %s (%s) ---\n", d.name, d.arch);
  std::printf("Global Memory: %lld MB\n", (long long)(d.global_mem_bytes >> 20));
  std::printf("LDS per Block: %lld KB\n", (long long)(d.lds_per_block_bytes >> 10));
  std::printf("LDS per CU: %lld KB\n", (long long)(d.lds_per_cu_bytes >> 10));
  std::printf("Registers per Block: %d\n", d.regs_per_block);
  std::printf("Registers per CU: %d\n", d.regs_per_cu);
  std::printf("L2 Cache Size: %lld KB\n", (long long)(d.l2_bytes >> 10));
  std::printf("Arch (major.minor): %d.%d\n", d.arch_major, d.arch_minor);
  std::printf("CU Count: %d\n", d.compute_units);
  std::printf("Max Threads per CU: %d\n", d.max_threads_per_cu);
  std::printf("Max Threads per Block: %d\n", d.max_threads_per_block);
  std::printf("Wavefront Size: %d\n", d.wavefront_size);
  std::printf("Clock: %d MHz\n", d.clock_khz / 1000);
  std::printf("Dense fp16/bf16 MFMA peak: %.1f TFLOP/s\n", d.fp16_dense_peak_tflops);
  std::printf("HBM peak: %.0f GB/s\n", d.hbm_peak_gbps);
  return 0;
}
