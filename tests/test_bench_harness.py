"""CPU tests of the benchmark harness: the result schema and row arithmetic
(fa_bench/schema.py, following benchmark/api/schema.py:3-34 and
benchmark/python/benchmark_pybind.py:74-118), the CLI's argument surface and
the fa_profile executable's command line (no kernel is launched here)."""
from __future__ import annotations

import os
import subprocess

import pytest

from fa_bench import schema
from fa_bench.schema import CSV_COLUMNS, csv_line, make_row, reference_flops, summarize

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PROFILE = os.path.join(REPO, "flash-attention_amd", "flash_attention_runtime", "fa_profile")


def test_schema_columns():
    assert len(CSV_COLUMNS) == 30 and len(set(CSV_COLUMNS)) == 30
    assert CSV_COLUMNS[:3] == ["mode", "kernel", "dtype"]
    assert CSV_COLUMNS[-1] == "run_id"


def test_reference_flop_count():
    # B*H*(4N^2 d + 6N^2): C3 = 1.0995e12 + 6*4*32*4096^2 -> 1.1124e12
    assert reference_flops(4, 32, 4096, 128) == 4 * 32 * (4 * 4096 ** 2 * 128 + 6 * 4096 ** 2)
    assert reference_flops(4, 32, 4096, 128, causal=True) == reference_flops(4, 32, 4096, 128) // 2
    assert schema.metric_flops(4, 32, 4096, 128) == 4.0 * 4 * 32 * 4096 ** 2 * 128


def test_summarize():
    s = summarize([1.0, 2.0, 3.0, 10.0])
    assert (s.mean, s.median, s.min, s.max) == (4.0, 2.5, 1.0, 10.0)
    assert s.stddev == pytest.approx(4.0825, rel=1e-4)
    assert summarize([2.0]).stddev == 0.0
    with pytest.raises(ValueError):
        summarize([])


def test_row_arithmetic():
    st = summarize([2.0, 2.0])
    meta = {"git_commit": "abc", "gpu_name": "gpu", "torch_version": "t", "cuda_version": "c",
            "run_id": "r1"}
    row = make_row(kernel="fa2_pybind", stats=st, baseline_mean=4.0, dtype="fp16", d_head=128,
                   seq_len=1024, batch_size=2, n_heads=4, warmups=1, repeats=2, stabilize=True,
                   baseline="pytorch", input_mode="random", elem_bytes=2, causal=False, meta=meta)
    assert set(row) == set(CSV_COLUMNS)
    flops = reference_flops(2, 4, 1024, 128)
    assert row["theoretical_flops"] == flops
    assert float(row["attn_tflops"]) == pytest.approx(flops / 2e-3 / 1e12, rel=1e-6)
    assert float(row["achieved_gflops"]) == pytest.approx(flops / 2e-3 / 1e9, rel=1e-6)
    assert row["rel_perf_pct"] == "200.00"  # baseline twice as slow
    assert row["io_bytes_est"] == 4 * 2 * 4 * 1024 * 128 * 2
    assert float(row["throughput_tokens_per_s"]) == pytest.approx(2 * 4 * 1024 / 2e-3, rel=1e-6)
    line = csv_line(row)
    assert line.split(",")[0] == "pybind" and line.split(",")[-1] == "r1"
    assert len(line.split(",")) == 30


def test_cli_arguments():
    from fa_bench.benchmark_pybind import parse_args

    a = parse_args([])
    assert (a.d_heads, a.seq_lens, a.n_heads, a.dtype, a.baseline) == ("128", "4096", 16,
                                                                        "fp16", "pytorch")
    a = parse_args(["--dtype", "bf16", "--causal", "--input_mode", "stress", "--csv"])
    assert a.dtype == "bf16" and a.causal and a.input_mode == "stress" and a.csv
    with pytest.raises(SystemExit):
        parse_args(["--dtype", "fp32"])


def test_profile_cli_usage():
    out = subprocess.run([PROFILE, "--help"], capture_output=True, text=True, timeout=60)
    assert out.returncode == 0
    assert "BxHxNxD" in out.stdout and "rocprof" in out.stdout and "c3" in out.stdout
    for bad in (["--mode", "ncu2"], ["--dtype", "fp32"], ["--bogus"], ["nosuchconfig"],
                ["1x2x3"], ["a", "b"]):
        r = subprocess.run([PROFILE, *bad], capture_output=True, text=True, timeout=60)
        assert r.returncode == 1, bad


PROBE = os.path.join(REPO, "flash-attention_amd", "flash_attention_runtime", "fa_mfma_probe")


def test_mfma_probe_cli_rejects_bad_arguments():
    """fa_mfma_probe validates its arguments before it touches a GPU."""
    for bad in (["--ms", "0"], ["--ms", "abc"], ["--ms", "5000"], ["--rounds", "0"], ["--bogus"],
                ["--ms"]):
        r = subprocess.run([PROBE, *bad], capture_output=True, text=True, timeout=60)
        assert r.returncode == 2, (bad, r.stdout, r.stderr)
        assert "usage" in r.stderr or "must be" in r.stderr
