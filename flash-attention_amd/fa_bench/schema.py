"""Result schema of the benchmark harness.

The column list is the reference's on-disk format
(benchmark/api/schema.py:3-34) so result files from both harnesses can be
merged by the same tooling; the row arithmetic follows
benchmark/python/benchmark_pybind.py:74-118.
"""
from __future__ import annotations

import statistics
from dataclasses import dataclass

CSV_COLUMNS = [
    "mode", "kernel", "dtype", "d_head", "seq_len", "batch_size", "n_heads", "warmups",
    "repeats", "stabilize", "baseline", "input_mode", "mean_ms", "median_ms", "min_ms",
    "max_ms", "stddev_ms", "rel_perf_pct", "attn_tflops", "theoretical_flops",
    "achieved_gflops", "throughput_tokens_per_ms", "throughput_tokens_per_s", "io_bytes_est",
    "est_bw_gbps", "git_commit", "gpu_name", "torch_version", "cuda_version", "run_id",
]


def reference_flops(batch: int, heads: int, seq_len: int, d_head: int, causal: bool = False) -> int:
    """The reference harness's count B*H*(4 N^2 d + 6 N^2) (benchmark_pybind.py:74-75,
    perf_metrics.cuh:140), halved for a causal run (the reference has none)."""
    f = batch * heads * (4 * seq_len * seq_len * d_head + 6 * seq_len * seq_len)
    return f // 2 if causal else f


def metric_flops(batch: int, heads: int, seq_len: int, d_head: int, causal: bool = False) -> float:
    """4*B*H*N^2*D, halved for causal: the metric this library is measured on."""
    f = 4.0 * batch * heads * seq_len * seq_len * d_head
    return f / 2 if causal else f


@dataclass
class Stats:
    mean: float
    median: float
    min: float
    max: float
    stddev: float


def summarize(samples_ms: list[float]) -> Stats:
    if not samples_ms:
        raise ValueError("no samples")
    return Stats(
        mean=statistics.mean(samples_ms),
        median=statistics.median(samples_ms),
        min=min(samples_ms),
        max=max(samples_ms),
        stddev=statistics.stdev(samples_ms) if len(samples_ms) > 1 else 0.0,
    )


def make_row(*, kernel: str, stats: Stats, baseline_mean: float, dtype: str, d_head: int,
             seq_len: int, batch_size: int, n_heads: int, warmups: int, repeats: int,
             stabilize: bool, baseline: str, input_mode: str, elem_bytes: int, causal: bool,
             meta: dict, mode: str = "pybind") -> dict:
    """One result row (all CSV_COLUMNS), values formatted as the reference
    formats them (benchmark_pybind.py:276-297)."""
    flops = reference_flops(batch_size, n_heads, seq_len, d_head, causal)
    tokens = batch_size * n_heads * seq_len
    io_bytes = 4 * batch_size * n_heads * seq_len * d_head * elem_bytes
    row = {
        "mode": mode,
        "kernel": kernel,
        "dtype": dtype,
        "d_head": d_head,
        "seq_len": seq_len,
        "batch_size": batch_size,
        "n_heads": n_heads,
        "warmups": warmups,
        "repeats": repeats,
        "stabilize": int(stabilize),
        "baseline": baseline,
        "input_mode": input_mode,
        "mean_ms": f"{stats.mean:.6f}",
        "median_ms": f"{stats.median:.6f}",
        "min_ms": f"{stats.min:.6f}",
        "max_ms": f"{stats.max:.6f}",
        "stddev_ms": f"{stats.stddev:.6f}",
        "rel_perf_pct": f"{100.0 * baseline_mean / stats.mean:.2f}",
        "attn_tflops": f"{flops / (stats.mean * 1e6) / 1e3:.6f}",
        "theoretical_flops": flops,
        "achieved_gflops": f"{flops / (stats.mean * 1e6):.6f}",
        "throughput_tokens_per_ms": f"{tokens / stats.mean:.6f}",
        "throughput_tokens_per_s": f"{tokens / stats.mean * 1e3:.6f}",
        "io_bytes_est": io_bytes,
        "est_bw_gbps": f"{io_bytes / (stats.mean * 1e6):.6f}",
    }
    for k in ("git_commit", "gpu_name", "torch_version", "cuda_version", "run_id"):
        row[k] = meta.get(k, "")
    return row


def csv_line(row: dict) -> str:
    return ",".join(str(row[c]) for c in CSV_COLUMNS)
