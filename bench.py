"""Benchmark of the MI355X FlashAttention-2 forward (BASELINE.json metric).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload C3]
                    [--no-cpu-baseline] [--all]

A step is one forward over one batch of synthetic input already resident in
HBM: flash_attention_runtime.forward(q, k, v, o) on the headline workload C3
(B=4, H=32, N=4096, D=128, fp16, non-causal; Q, K, V ~ N(0, 1) from seed
1234 + 100003*2, the reference's convention in
benchmark/python/input_data.py:11-30).  W untimed warmup steps, then K steps
timed by two HIP events on the stream the kernel is launched on, bracketed by
device synchronisation.  FLOPs per step = 4*B*H*N^2*D (halved for causal).

Order of the run: the CPU baseline (host only), then the cold-cache figure
(COLD_LAUNCHES launches of the same workload on the same tensors, each after
a 512 MiB cache flush), then the W warmup and K timed steps, with no idle gap
between them.  On a fresh MI355X the power controller takes about 25
back-to-back C3 launches to settle after the GPU starts from idle: the first
launch runs at a high clock, launches 2-6 at a low one (1.2 ms instead of
0.96 ms) and the next 20 recover step by step.  The cold-cache launches come
first so that the timed steps measure the settled clock, which is what a
caller issuing attention back to back sees; the JSON line reports how many
launches of the workload preceded the timed region ("launches_before_timed").

Prints one JSON line with the metric, the roofline of the kernel (MFMA bound,
against MI355X's published dense fp16/bf16 peak of 2.5 PFLOP/s) and a CPU
baseline: the reference's CPU path (cpu_reference_attention,
benchmark/cpp/correctness_v6.cu:23-72, restated in oracle/attn_oracle.c)
timed on a bounded sample of rows of the same workload on the host cores.

--all additionally times every BASELINE config and prints a table to stderr.
--split-table times few-head shapes with and without split-KV instead.
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

REPO_ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO_ROOT, "flash-attention_amd"))  # runtime + fa_bench
sys.path.insert(0, REPO_ROOT)

PEAK_FP16_TFLOPS = 2500.0  # MI355X published dense fp16/bf16 MFMA peak
PEAK_HBM_GBPS = 8000.0

# id: (B, H, N, D, dtype, causal, qk_sigma, case_index)  — BASELINE.json configs
WORKLOADS = {
    "C2": (4, 16, 1024, 64, "fp16", False, 1.0, 1),
    "C3": (4, 32, 4096, 128, "fp16", False, 1.0, 2),
    "C4": (2, 32, 8192, 128, "bf16", True, 1.0, 3),
    "C5": (1, 16, 16384, 128, "fp16", True, 3.0, 4),
    "C5r": (1, 16, 3000, 128, "fp16", True, 3.0, 5),
}
# Few-head shapes that leave most CUs idle unsplit (the target of split-KV;
# not BASELINE configs): timed with and without the split by --split-table.
SPLIT_SHAPES = {
    "S1": (1, 1, 4096, 128, "fp16", False, 1.0, 11),
    "S2": (1, 4, 8192, 128, "fp16", True, 1.0, 12),
    "S3": (1, 8, 3000, 128, "fp16", True, 3.0, 13),
    "S4": (1, 2, 8192, 128, "bf16", True, 1.0, 14),
    "S5": (2, 4, 2048, 64, "fp16", False, 1.0, 15),
}
TRAFFIC_FILE = os.path.join(REPO_ROOT, "profiles", "fa_fwd_C3_traffic.json")


def flops(B, H, N, D, causal):
    f = 4.0 * B * H * N * N * D
    return f / 2 if causal else f


def make_inputs(torch, name, device, input_mode="random"):
    from fa_bench.input_data import generate_qkv

    B, H, N, D, dtype, causal, sigma, case = {**WORKLOADS, **SPLIT_SHAPES}[name]
    td = {"fp16": torch.float16, "bf16": torch.bfloat16}[dtype]
    q, k, v, _ = generate_qkv(batch_size=B, n_heads=H, seq_len=N, d_head=D, dtype=td,
                              device=device, input_mode=input_mode, seed=1234, case_index=case,
                              qk_sigma=sigma)
    return (q, k, v), causal


def time_workload(torch, fa, name, steps, warmup, input_mode="random", split_kv=True,
                  tensors=None):
    if tensors is None:
        (q, k, v), causal = make_inputs(torch, name, "cuda", input_mode)
        o = torch.empty_like(q)
    else:
        q, k, v, o, causal = tensors
    for _ in range(warmup):
        fa.forward(q, k, v, o, causal=causal, split_kv=split_kv)
    stream = torch.cuda.current_stream()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(steps):
        fa.forward(q, k, v, o, causal=causal, split_kv=split_kv)
    stop.record(stream)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    ms = start.elapsed_time(stop) / steps
    B, H, N, D = q.shape
    tflops = flops(B, H, N, D, causal) / (ms * 1e-3) / 1e12
    return ms, tflops, wall_ms


def gemm_ceiling(torch, steps, warmup):
    """Times square torch.matmul GEMMs (hipBLASLt on ROCm) on N(0,1) and on
    constant operands.  MI355X clocks depend on the data the matrix cores
    toggle, so the random-data figure is the relevant ceiling for attention
    on random inputs.  Prints one JSON line per case."""
    for dt_name, dt in (("fp16", torch.float16), ("bf16", torch.bfloat16)):
        for n in (8192, 16384):
            for data in ("randn", "ones"):
                g = torch.Generator(device="cuda")
                g.manual_seed(7)
                if data == "randn":
                    a = torch.randn((n, n), generator=g, device="cuda").to(dt)
                    b = torch.randn((n, n), generator=g, device="cuda").to(dt)
                else:
                    a = torch.ones((n, n), device="cuda", dtype=dt)
                    b = torch.ones((n, n), device="cuda", dtype=dt)
                c = torch.empty((n, n), device="cuda", dtype=dt)
                for _ in range(min(max(warmup, 3), 20)):  # GEMMs of ms each
                    torch.matmul(a, b, out=c)
                reps = max(5, min(steps, 50))
                start = torch.cuda.Event(enable_timing=True)
                stop = torch.cuda.Event(enable_timing=True)
                torch.cuda.synchronize()
                start.record()
                for _ in range(reps):
                    torch.matmul(a, b, out=c)
                stop.record()
                torch.cuda.synchronize()
                ms = start.elapsed_time(stop) / reps
                print(json.dumps({"gemm": f"{n}x{n}x{n}", "dtype": dt_name, "data": data,
                                  "ms": round(ms, 4),
                                  "tflops": round(2.0 * n ** 3 / (ms * 1e-3) / 1e12, 1)}),
                      flush=True)
                del a, b, c


COLD_LAUNCHES = 50


def time_cold(torch, fa, q, k, v, o, causal, steps):
    """Per-launch time with the last-level caches flushed before every launch
    (a 512 MiB write; MI355X's L2 + MALL hold 256 MiB), each launch bracketed
    by its own HIP events (benchmark_pybind.py:135-176 does the same with
    100 MiB).  Returns the median time, its TFLOP/s and the number of
    launches made (steps + 1)."""
    flush = torch.empty(512 << 20, dtype=torch.int8, device="cuda")
    fa.forward(q, k, v, o, causal=causal)
    times = []
    for _ in range(steps):
        flush.zero_()
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        fa.forward(q, k, v, o, causal=causal)
        b.record()
        torch.cuda.synchronize()
        times.append(a.elapsed_time(b))
    times.sort()
    ms = times[len(times) // 2]
    B, H, N, D = q.shape
    return ms, flops(B, H, N, D, causal) / (ms * 1e-3) / 1e12, steps + 1


SHAPE_LIBS = {
    "product": os.path.join(REPO_ROOT, "flash-attention_amd", "flash_attention_runtime", "libfa_mi355x.so"),
    "mfma32": os.path.join(REPO_ROOT, "flash-attention_amd", "flash_attention_runtime",
                           "libfa_mi355x_mfma32.so"),
}


def time_abi(torch, lib_name, name, steps, warmup, rounds):
    """Times one workload through the C ABI (fa_fwd) of the product library
    (D = 128 on the 16x16x32 MFMA kernel) or of the test-only build that keeps
    the 32x32x16 form everywhere (libfa_mi355x_mfma32.so): W launches, then
    `rounds` groups of K launches, each timed by HIP events.  Returns the
    per-launch ms of each group."""
    import ctypes

    sys.path.insert(0, os.path.join(REPO_ROOT, "tests"))
    import abi_ctypes as A

    lib = A.load(SHAPE_LIBS[lib_name])
    (q, k, v), causal = make_inputs(torch, name, "cuda")
    o = torch.empty_like(q)
    p = A.params_from_tensors(q, k, v, o, None, causal)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for _ in range(warmup):
        assert lib.fa_fwd(ctypes.byref(p), stream) == 0, lib.fa_last_error()
    out = []
    for _ in range(rounds):
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(steps):
            lib.fa_fwd(ctypes.byref(p), stream)
        b.record()
        torch.cuda.synchronize()
        out.append(a.elapsed_time(b) / steps)
    return out


def cpu_baseline(name, budget_s=15.0):
    """Times the reference CPU path (oracle_ref_online_f32: fp32 online softmax
    with expf, one query row at a time) on the first rows of the workload, on
    all host threads OpenMP gives it; returns TFLOP/s of the same metric."""
    import numpy as np
    import torch

    from oracle import oracle as O

    B, H, N, D, dtype, causal, sigma, case = WORKLOADS[name]
    (q, k, v), _ = make_inputs(torch, name, "cpu")
    flat = [t.reshape(1, B * H, N, D) for t in (q, k, v)]
    threads = O.num_threads()
    scale = 1.0 / math.sqrt(D)

    def run(rows):
        nh = min(B * H, -(-rows // N))  # heads the rows span
        qn, kn, vn = (t[:, :nh].float().numpy() for t in flat)
        t0 = time.perf_counter()
        O.ref_online_f32(qn, kn, vn, scale, causal, 0, rows)
        return time.perf_counter() - t0, nh

    # calibrate (grow the sample until it takes >= 0.3 s), then size to budget_s
    rows = max(threads, 8)
    while True:
        dt, _ = run(rows)
        if dt >= 0.3 or rows >= B * H * N:
            break
        rows = min(B * H * N, rows * 4)
    rows = int(min(B * H * N, max(rows, rows * budget_s / max(dt, 1e-6))))
    dt, nh = run(rows)
    # A whole workload shorter than the budget is timed repeatedly.
    reps = 1
    while dt < budget_s * 0.6 and rows == B * H * N and reps < 8:
        dt += run(rows)[0]
        reps += 1
    # FLOPs of those rows under the metric's convention (4*N*D per row,
    # halved-on-average for causal is not applied to a row sample: use the
    # visible key count of each row).
    if causal:
        keys = sum(min(N, (r % N) + 1) for r in range(rows))
    else:
        keys = rows * N
    f = 4.0 * keys * D * reps
    return {
        "value": f / dt / 1e12,
        "unit": "TFLOPS",
        "cores": threads,
        "kind": "port",
        "sample": (f"first {rows} query rows (the first {nh} of {B * H} heads) of {name} "
                   f"({keys * D * 4:.3g} flop) x {reps} run(s), "
                   f"fp32 online softmax with expf as correctness_v6.cu:23-72, "
                   f"{threads} OpenMP threads, {dt:.1f} s"),
    }


def cpu_torch_baseline(name, budget_s=5.0):
    """torch's CPU scaled_dot_product_attention in fp32 on whole heads of the
    workload (the reference harness's pytorch baseline, benchmark_pybind.py:
    129-132, run on the host), all torch threads; returns TFLOP/s."""
    import torch

    B, H, N, D, dtype, causal, sigma, case = WORKLOADS[name]
    (q, k, v), _ = make_inputs(torch, name, "cpu")
    qf, kf, vf = (t.reshape(B * H, 1, N, D).float() for t in (q, k, v))
    sdpa = torch.nn.functional.scaled_dot_product_attention
    per_head = flops(1, 1, N, D, causal)
    t0 = time.perf_counter()
    sdpa(qf[:1], kf[:1], vf[:1], is_causal=causal)
    dt1 = max(time.perf_counter() - t0, 1e-4)
    heads = int(max(1, min(B * H, budget_s / dt1)))
    t0 = time.perf_counter()
    for i in range(heads):
        sdpa(qf[i:i + 1], kf[i:i + 1], vf[i:i + 1], is_causal=causal)
    dt = time.perf_counter() - t0
    return {
        "value": per_head * heads / dt / 1e12,
        "unit": "TFLOPS",
        "cores": torch.get_num_threads(),
        "kind": "torch-cpu",
        "sample": f"{heads} of {B * H} heads of {name}, fp32 SDPA, {dt:.1f} s",
    }


def main():
    ap = argparse.ArgumentParser(description="MI355X FlashAttention-2 forward benchmark")
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="C3", choices=sorted(WORKLOADS))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--all", action="store_true", help="also time every config (stderr table)")
    ap.add_argument("--split-table", action="store_true",
                    help="instead of the metric, time the few-head shapes with and without "
                         "split-KV (stderr table)")
    ap.add_argument("--input-mode", default="random", choices=["random", "structured", "stress"],
                    help="input values (the headline metric is quoted on random)")
    ap.add_argument("--gemm-ceiling", action="store_true",
                    help="instead of attention, time torch.matmul (hipBLASLt) fp16/bf16 GEMMs on "
                         "N(0,1) and on constant data: the data-dependent MFMA ceiling of the box")
    ap.add_argument("--mfma-shapes", action="store_true",
                    help="instead of the metric, time --workload (or C3 and C4) through the C ABI of "
                         "the product library and of the 32x32x16 build (--shape-lib picks one), "
                         "alternating (stderr table)")
    ap.add_argument("--shape-lib", choices=sorted(SHAPE_LIBS), default=None,
                    help="with --mfma-shapes: time only this library (for counter runs)")
    ap.add_argument("--copy-mib", type=int, default=0,
                    help="instead of attention, time a plain device copy of this many MiB "
                         "(calibrates the FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "the forward shards over (batch, head) with no communication, so N GPUs "
              "would each run this same single-GPU benchmark on their share.", file=sys.stderr)
        sys.exit(2)

    import torch

    import flash_attention_runtime as fa

    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)

    if args.copy_mib:
        n = args.copy_mib * (1 << 20) // 4
        src = torch.randn(n, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(args.warmup):
            dst.copy_(src)
        start = torch.cuda.Event(enable_timing=True)
        stop = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        start.record()
        for _ in range(args.steps):
            dst.copy_(src)
        stop.record()
        torch.cuda.synchronize()
        ms = start.elapsed_time(stop) / args.steps
        print(json.dumps({"copy_bytes_read": n * 4, "copy_bytes_written": n * 4, "ms": ms,
                          "GBps_read_plus_write": 2 * n * 4 / (ms * 1e-3) / 1e9}), flush=True)
        return

    if args.gemm_ceiling:
        gemm_ceiling(torch, args.steps, args.warmup)
        return

    if args.mfma_shapes:
        libs = [args.shape_lib] if args.shape_lib else ["mfma32", "product"]
        names = [args.workload] if "--workload" in sys.argv else ["C3", "C4"]
        print(f"{'cfg':5s} {'library':8s} {'ms per launch (rounds)':>40s} {'best TFLOPS':>12s}",
              file=sys.stderr, flush=True)
        for wn in names:
            B, H, N, D, dtype, causal, _, _ = WORKLOADS[wn]
            res = {ln: [] for ln in libs}
            for _ in range(2):  # alternate the libraries, twice
                for ln in libs:
                    res[ln] += time_abi(torch, ln, wn, args.steps, args.warmup, 2)
            for ln in libs:
                best = min(res[ln])
                print(f"{wn:5s} {ln:8s} {' '.join(f'{t:.4f}' for t in res[ln]):>40s} "
                      f"{flops(B, H, N, D, causal) / (best * 1e-3) / 1e12:12.1f}",
                      file=sys.stderr, flush=True)
        return

    if args.split_table:
        print(f"{'shape':5s} {'B':>2s} {'H':>3s} {'N':>6s} {'D':>4s} {'dtype':>5s} {'mask':>7s} "
              f"{'unsplit ms':>11s} {'split ms':>9s} {'speed-up':>9s} {'split TFLOPS':>13s}",
              file=sys.stderr, flush=True)
        for sn, (B, H, N, D, dt, causal, _, _) in SPLIT_SHAPES.items():
            u_ms, _, _ = time_workload(torch, fa, sn, args.steps, args.warmup, args.input_mode,
                                       split_kv=False)
            s_ms, s_tf, _ = time_workload(torch, fa, sn, args.steps, args.warmup,
                                          args.input_mode, split_kv=True)
            print(f"{sn:5s} {B:2d} {H:3d} {N:6d} {D:4d} {dt:>5s} "
                  f"{'causal' if causal else 'none':>7s} {u_ms:11.4f} {s_ms:9.4f} "
                  f"{u_ms / s_ms:8.2f}x {s_tf:13.1f}", file=sys.stderr, flush=True)
        return

    name = args.workload
    B, H, N, D, dtype, causal, sigma, case = WORKLOADS[name]
    # Host-only baselines first: the GPU idles meanwhile, and nothing idles it
    # between the cold-cache launches and the timed steps.
    cpu = None if args.no_cpu_baseline else cpu_baseline(name)
    cpu_torch = None if args.no_cpu_baseline else cpu_torch_baseline(name)
    (q, k, v), _ = make_inputs(torch, name, "cuda", args.input_mode)
    o = torch.empty_like(q)
    cold_ms, cold_tflops, n_cold = time_cold(torch, fa, q, k, v, o, causal, COLD_LAUNCHES)
    ms, tflops, wall_ms = time_workload(torch, fa, name, args.steps, args.warmup,
                                        tensors=(q, k, v, o, causal))
    info = fa.device_info(0)

    traffic = None
    if os.path.exists(TRAFFIC_FILE) and name == "C3":
        with open(TRAFFIC_FILE) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")

    if args.all:
        print(f"{'cfg':5s} {'ms':>9s} {'TFLOPS':>9s} {'%peak':>7s}", file=sys.stderr)
        for wn in WORKLOADS:
            wms, wtf, _ = time_workload(torch, fa, wn, max(10, args.steps // 2), args.warmup,
                                        args.input_mode)
            print(f"{wn:5s} {wms:9.4f} {wtf:9.1f} {100 * wtf / PEAK_FP16_TFLOPS:6.1f}%",
                  file=sys.stderr, flush=True)


    line = {
        "metric": "fwd TFLOPS + % of FP16 MFMA peak, B4 H32 N4096 D128 fp16 (1 GPU)",
        "value": round(tflops, 2),
        "unit": "TFLOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype,
        "data": (f"synthetic, resident in HBM: {args.input_mode} mode"
                 + (" (Q,K,V ~ N(0,1), seed 1234 + 100003*case)" if args.input_mode == "random" else "")),
        "config": {
            "workload": f"{name}: B={B} H={H} N={N} D={D} {dtype} "
                        f"{'causal' if causal else 'non-causal'} FA2 forward",
            "batch": B, "heads": H, "seq_len": N, "head_dim": D, "causal": causal,
            "parallelism": "single GPU",
        },
        "pct_of_peak": round(100.0 * tflops / PEAK_FP16_TFLOPS, 2),
        "roofline": {
            "bound": "mfma",
            "achieved": round(tflops, 2),
            "peak": PEAK_FP16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(tflops / PEAK_FP16_TFLOPS, 4),
            "traffic": traffic,
        },
        "cpu_baseline": cpu,
        "cpu_baseline_torch": cpu_torch,
        "cold": {"ms_per_step": round(cold_ms, 5), "tflops": round(cold_tflops, 2),
                 "note": f"median of {COLD_LAUNCHES} launches, each after a 512 MiB cache flush, "
                         "run before the warmup steps"},
        "launches_before_timed": n_cold + args.warmup,
        "device": {k: info[k] for k in ("arch", "compute_units", "clock_khz",
                                        "fp16_dense_peak_tflops")},
        "wall_ms_timed_region": round(wall_ms, 2),
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
