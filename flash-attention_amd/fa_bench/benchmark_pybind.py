"""Benchmark of the Python entry point, with the reference harness's options
and result format.

Replaces benchmark/python/benchmark_pybind.py (CLI :179-229, timing
:135-176, rows :276-297): for each (d_head, seq_len) it times
flash_attention_runtime.forward_timed on generated inputs and, as the
100 % line, torch's own scaled_dot_product_attention restricted to its flash
backend on the same tensors.  Rows use the 30-column schema of
fa_bench/schema.py; they are printed as a table (default) or CSV (--csv) and
saved to --out_csv unless --no_save.  --result_json writes a run summary.

    python -m fa_bench.benchmark_pybind --d_heads 64,128 --seq_lens 1024,4096 \
        --batch_size 4 --n_heads 32 --dtype fp16 --csv --no_save

Differences from the reference harness: --dtype is fp16 or bf16 (the
reference defaults to fp32, which its own extension rejects), --causal is
supported, and the cache flush between repeats writes 512 MiB (the MI355X
last-level cache is 256 MiB) instead of 100 MiB.  The FLOP columns keep the
reference's count B*H*(4 N^2 d + 6 N^2) (halved for causal).
"""
from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import time
from datetime import datetime
from pathlib import Path

import torch

_PKG = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if _PKG not in sys.path:
    sys.path.insert(0, _PKG)

import flash_attention_runtime as fa  # noqa: E402
from fa_bench.input_data import MODES, generate_qkv  # noqa: E402
from fa_bench.schema import CSV_COLUMNS, csv_line, make_row, summarize  # noqa: E402

# benchmark_pybind.py:23-30: batch size per seq_len when --batch_size is 0
BATCH_SIZE_FOR_SEQ_LEN = {512: 16, 1024: 16, 2048: 16, 4096: 16, 8192: 8, 16384: 4}
FLUSH_BYTES = 512 << 20


def parse_args(argv=None):
    p = argparse.ArgumentParser(description="Benchmark the flash_attention_runtime entry point")
    p.add_argument("--d_heads", default="128", help="comma separated head dims")
    p.add_argument("--seq_lens", default="4096", help="comma separated seq lens")
    p.add_argument("--batch_size", type=int, default=8, help="0: per-seq_len default table")
    p.add_argument("--n_heads", type=int, default=16)
    p.add_argument("--warmups", type=int, default=10)
    p.add_argument("--repeats", type=int, default=50)
    p.add_argument("--no_stabilize", action="store_true", help="no cache flush between repeats")
    p.add_argument("--csv", action="store_true", help="print CSV rows instead of a table")
    p.add_argument("--out_csv", default="", help="default: profile_results/pybind_<time>.csv")
    p.add_argument("--no_save", action="store_true")
    p.add_argument("--result_json", default="", help="also write a run summary JSON here")
    p.add_argument("--baseline", default="pytorch", choices=["pytorch", "fa2_pybind"],
                   help="kernel used as 100%% for rel_perf_pct")
    p.add_argument("--dtype", default="fp16", choices=["fp16", "bf16"])
    p.add_argument("--causal", action="store_true")
    p.add_argument("--input_mode", default="random", choices=list(MODES))
    p.add_argument("--seed", type=int, default=1234)
    p.add_argument("--replay_dir", default="benchmark/data/replay")
    p.add_argument("--replay_file", default="")
    return p.parse_args(argv)


def git_commit() -> str:
    try:
        return subprocess.check_output(["git", "rev-parse", "HEAD"], cwd=_PKG, text=True,
                                       stderr=subprocess.DEVNULL).strip()
    except Exception:
        return "unknown"


def run_meta() -> dict:
    return {
        "git_commit": git_commit(),
        "gpu_name": torch.cuda.get_device_name(0).replace(",", " "),
        "torch_version": torch.__version__,
        "cuda_version": ("hip-" + torch.version.hip) if torch.version.hip else
                        (torch.version.cuda or "unknown"),
        "run_id": datetime.now().strftime("%Y%m%d_%H%M%S") + f"_{os.getpid()}",
    }


def time_samples(fn, warmups: int, repeats: int, flush_buf) -> list[float]:
    """Per-repeat kernel time in ms.  fn returns either a tensor (timed here
    with events) or (tensor, ms) from forward_timed (its own event pair)."""
    for _ in range(warmups):
        fn()
    torch.cuda.synchronize()
    out = []
    for _ in range(repeats):
        if flush_buf is not None:
            flush_buf.zero_()
            torch.cuda._sleep(1_000_000)
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        a.record()
        r = fn()
        b.record()
        torch.cuda.synchronize()
        out.append(float(r[1]) if isinstance(r, tuple) else float(a.elapsed_time(b)))
    return out


def torch_flash_fn(q, k, v, causal):
    """torch SDPA restricted to its flash backend (no silent fallback to the
    math path); returns None if that backend cannot run these inputs."""
    from torch.nn.attention import SDPBackend, sdpa_kernel

    def fn():
        with sdpa_kernel([SDPBackend.FLASH_ATTENTION]):
            return torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=causal)

    try:
        fn()
        torch.cuda.synchronize()
    except RuntimeError as e:
        print(f"note: torch flash SDPA unavailable here ({str(e).splitlines()[0]})")
        return None
    return fn


def print_table(title: str, rows: list[dict]) -> None:
    head = ["kernel", "d_head", "seq_len", "mean_ms", "attn_tflops", "rel_perf_pct",
            "est_bw_gbps"]
    cells = [[str(r[h]) for h in head] for r in rows]
    w = [max(len(h), *(len(c[i]) for c in cells)) for i, h in enumerate(head)]
    print(title)
    print(" | ".join(h.ljust(w[i]) for i, h in enumerate(head)))
    print("-+-".join("-" * x for x in w))
    for c in cells:
        print(" | ".join(c[i].ljust(w[i]) for i in range(len(head))))
    print()


def main(argv=None) -> list[dict]:
    args = parse_args(argv)
    if not torch.cuda.is_available():
        raise RuntimeError("a GPU is required")
    meta = run_meta()
    td = {"fp16": torch.float16, "bf16": torch.bfloat16}[args.dtype]
    print(f"GPU: {meta['gpu_name']}  torch={meta['torch_version']} {meta['cuda_version']} "
          f"commit={meta['git_commit'][:12]}  library={fa.version()}")
    print(f"warmups={args.warmups} repeats={args.repeats} stabilize={not args.no_stabilize} "
          f"baseline={args.baseline} dtype={args.dtype} causal={args.causal} "
          f"input_mode={args.input_mode} seed={args.seed}\n")
    flush = None if args.no_stabilize else torch.empty(FLUSH_BYTES, dtype=torch.int8,
                                                        device="cuda")
    rows: list[dict] = []
    header_done = False
    case = 0
    for d in (int(x) for x in args.d_heads.split(",")):
        for n in (int(x) for x in args.seq_lens.split(",")):
            if d not in (64, 128):
                print(f"skip d_head={d}: supported head dims are 64 and 128")
                continue
            bsz = args.batch_size if args.batch_size > 0 else BATCH_SIZE_FOR_SEQ_LEN.get(n, 4)
            q, k, v, path = generate_qkv(batch_size=bsz, n_heads=args.n_heads, seq_len=n,
                                         d_head=d, dtype=td, device="cuda",
                                         input_mode=args.input_mode, seed=args.seed,
                                         case_index=case, replay_dir=args.replay_dir,
                                         replay_file=args.replay_file)
            case += 1
            if path is not None:
                print(f"replay input: {path}")
            o = torch.empty_like(q)
            stats = {"fa2_pybind": summarize(time_samples(
                lambda: fa.forward_timed(q, k, v, o, causal=args.causal),
                args.warmups, args.repeats, flush))}
            tfn = torch_flash_fn(q, k, v, args.causal)
            if tfn is not None:
                stats["pytorch"] = summarize(time_samples(tfn, args.warmups, args.repeats, flush))
            base = args.baseline if args.baseline in stats else "fa2_pybind"
            case_rows = [
                make_row(kernel=name, stats=st, baseline_mean=stats[base].mean,
                         dtype=args.dtype, d_head=d, seq_len=n, batch_size=bsz,
                         n_heads=args.n_heads, warmups=args.warmups, repeats=args.repeats,
                         stabilize=not args.no_stabilize, baseline=args.baseline,
                         input_mode=args.input_mode, elem_bytes=2, causal=args.causal,
                         meta=meta)
                for name, st in stats.items()
            ]
            rows.extend(case_rows)
            if args.csv:
                if not header_done:
                    print(",".join(CSV_COLUMNS))
                    header_done = True
                for r in case_rows:
                    print(csv_line(r), flush=True)
            else:
                print_table(f"--- d_head={d} seq_len={n} batch={bsz} heads={args.n_heads} ---",
                            case_rows)
            del q, k, v, o
    out_csv = None
    if not args.no_save:
        out_csv = Path(args.out_csv) if args.out_csv else (
            Path("profile_results") / f"pybind_{meta['run_id']}.csv")
        out_csv.parent.mkdir(parents=True, exist_ok=True)
        with out_csv.open("w", encoding="utf-8") as f:
            f.write(",".join(CSV_COLUMNS) + "\n")
            for r in rows:
                f.write(csv_line(r) + "\n")
        print(f"saved csv: {out_csv}")
    if args.result_json:
        summary = {"run_id": meta["run_id"], "results_csv": str(out_csv) if out_csv else None,
                   "rows": len(rows), "args": vars(args), "meta": meta,
                   "finished": time.strftime("%Y-%m-%dT%H:%M:%S")}
        Path(args.result_json).write_text(json.dumps(summary, indent=2), encoding="utf-8")
    return rows


if __name__ == "__main__":
    main()
