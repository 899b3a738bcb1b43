"""The benchmark harness on the GPU: the pybind benchmark CLI
(fa_bench/benchmark_pybind.py) and the C++ fa_profile executable, at small
shapes, produce well-formed rows in the reference's formats."""
from __future__ import annotations

import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PROFILE = os.path.join(REPO, "flash-attention_amd", "flash_attention_runtime", "fa_profile")


def test_benchmark_pybind_rows(tmp_path, capsys):
    from fa_bench.benchmark_pybind import main
    from fa_bench.schema import CSV_COLUMNS

    print("case benchmark_pybind small", flush=True)
    out_csv = tmp_path / "r.csv"
    rows = main(["--d_heads", "64,128", "--seq_lens", "256", "--batch_size", "1", "--n_heads",
                 "2", "--warmups", "1", "--repeats", "3", "--csv", "--out_csv", str(out_csv),
                 "--result_json", str(tmp_path / "result.json")])
    kernels = {r["kernel"] for r in rows}
    assert "fa2_pybind" in kernels
    assert len([r for r in rows if r["kernel"] == "fa2_pybind"]) == 2
    for r in rows:
        assert float(r["mean_ms"]) > 0 and float(r["attn_tflops"]) > 0
    lines = out_csv.read_text().strip().splitlines()
    assert lines[0] == ",".join(CSV_COLUMNS)
    assert len(lines) == 1 + len(rows)
    assert all(len(ln.split(",")) == 30 for ln in lines)
    assert (tmp_path / "result.json").exists()


@pytest.mark.parametrize("extra", [[], ["--dtype", "bf16", "--causal"]])
def test_fa_profile_csv_line(extra):
    print(f"case fa_profile {extra}", flush=True)
    r = subprocess.run([PROFILE, "2x2x300x64", "--warmup-iters", "1", "--benchmark-iters", "3",
                        *extra], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    csv = [ln for ln in r.stdout.splitlines() if ln.startswith("CSV,")]
    assert len(csv) == 1
    f = csv[0].split(",")
    assert len(f) == 13
    assert f[1:5] == ["2", "2", "300", "64"]
    assert float(f[5]) > 0 and float(f[6]) > 0


def test_device_info_mi355x(fa):
    """The device query behind %-of-peak figures (replaces
    utils/get_gpu_hardware_param.cu): gfx950 with 256 CUs, the dense fp16
    MFMA peak derived from CUs x clock x 4096, and the published HBM rate."""
    print("case device_info", flush=True)
    info = fa.device_info(0)
    assert info["arch"].startswith("gfx950")
    assert info["name"]
    assert info["compute_units"] == 256
    expect = info["compute_units"] * info["clock_khz"] * 1e3 * 4096 / 1e12
    assert abs(info["fp16_dense_peak_tflops"] - expect) < 1e-6 * expect
    assert 2000 < info["fp16_dense_peak_tflops"] < 3000
    assert info["hbm_peak_gbps"] == 8000.0
    assert info["lds_per_cu_bytes"] >= 64 * 1024


PROBE = os.path.join(REPO, "flash-attention_amd", "flash_attention_runtime", "fa_mfma_probe")


def test_mfma_probe_reaches_formula_peak():
    """The MFMA-only probe: with low-toggle operands and one wave per SIMD the
    matrix cores must run near the CUs x clock x 4096 figure the benchmark
    divides by (a short run, before the power limiter settles)."""
    print("case fa_mfma_probe", flush=True)
    r = subprocess.run([PROBE, "--ms", "2", "--rounds", "1"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stderr
    rows = {}
    for ln in r.stdout.splitlines():
        f = ln.split()
        if len(f) >= 4 and f[0] in ("ones", "N(0,1)") and f[1] in ("1", "2"):
            rows[(f[0], int(f[1]))] = (float(f[2]), float(f[3].rstrip("%")))
    assert set(rows) == {("ones", 1), ("ones", 2), ("N(0,1)", 1), ("N(0,1)", 2)}
    assert rows[("ones", 1)][1] > 85.0, rows
    for tflops, pct in rows.values():
        assert 0.0 < pct <= 101.0 and tflops > 0.0


def test_bench_split_table():
    """bench.py --split-table times every few-head shape with and without
    split-KV; the split must not lose clearly on any of them (it measured
    1.26-2.7x faster; the bar leaves room for launch-to-launch noise of the
    short shapes on any box)."""
    import sys

    print("case bench --split-table", flush=True)
    r = subprocess.run([sys.executable, os.path.join(REPO, "bench.py"), "--split-table",
                        "--steps", "10", "--warmup", "2"], capture_output=True, text=True,
                       timeout=240)
    assert r.returncode == 0, r.stderr[-2000:]
    rows = [ln.split() for ln in r.stderr.splitlines() if ln[:2] in ("S1", "S2", "S3", "S4", "S5")]
    print("\n".join(" ".join(x) for x in rows), flush=True)
    assert [x[0] for x in rows] == ["S1", "S2", "S3", "S4", "S5"]
    for x in rows:
        unsplit, split = float(x[7]), float(x[8])
        assert unsplit > 0 and split > 0
        assert split < 1.15 * unsplit, x
