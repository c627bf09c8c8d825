"""Single-shape decode-attention microbenchmark (restates reference benchmarks/microbench.py).

    python -m flashspec_amd.microbench --backend triton_paged --batch 8 --heads 32 \\
        --seq-len 4096 --head-dim 128 --iters 50 --warmup 10 --repeats 20 --json

Same CLI, input draw order (q, k, v from one seeded generator), length patterns,
timing method (events around ``iters`` calls, median over ``repeats``) and JSON keys
as the reference (microbench.py:90-179, 406-631).  ``triton_*`` backends run the
HIP kernels.  Profiling uses rocprofv3 instead of Nsight Compute: ``--profile-rocprof``
re-runs this benchmark under ``rocprofv3`` in a child process and backfills the
``measured_*`` fields; the reference's ``nsight_compute_*`` keys are kept for schema
compatibility and hold the equivalent rocprofv3 commands.
"""

from __future__ import annotations

import argparse
import glob
import json
import os
import sqlite3
import statistics
import subprocess
import sys
import tempfile
from pathlib import Path
from time import perf_counter
from typing import Callable

import numpy as np
import torch

from . import (
    PagedKVCache,
    fused_dequant_attention,
    fused_dequant_attention_triton,
    paged_quant_attention,
    paged_quant_attention_triton,
    quantize_int8_per_block,
    reference_attention,
)
from .runtime import device_name, resolve_device, resolve_dtype, synchronize
from .triton_utils import HAS_TRITON

DTYPE_CHOICES = ["auto", "float16", "fp16", "bfloat16", "bf16", "float32", "fp32"]
# Kernels a backend's step launches (rocprofv3 kernel names, e.g.
# "void fs::decode_rows_kernel<128, __half, true, 0, 0>(fs::DecodeParams)"): the tiled decode kernel
# (template <head_dim layout, q type, paged, quant mode, value format>), the generic one and the
# split merge.
KERNEL_REGEX = {
    "triton_fused": r"decode_rows_kernel<[0-9]+, [^,]+, false[,>]|decode_generic_kernel<[^,]+, false[,>]|"
                    r"combine_splits",
    "triton_paged": r"decode_rows_kernel<[0-9]+, [^,]+, true[,>]|decode_generic_kernel<[^,]+, true[,>]|"
                    r"combine_splits",
}
# gfx950's FETCH_SIZE expression counts half of the bytes a plain device copy reads
# (calibration in profiles/paged_decode_b8h32s4096d128_pmc.json); WRITE_SIZE is exact.
FETCH_SIZE_SCALE = 2.0
PEAK_HBM_GBPS = 8000.0


def _percentile(values: list[float], pct: float) -> float:
    if not values:
        return 0.0
    ordered = sorted(values)
    if len(ordered) == 1:
        return ordered[0]
    pos = (len(ordered) - 1) * pct / 100.0
    lo = int(pos)
    hi = min(lo + 1, len(ordered) - 1)
    return ordered[lo] * (1.0 - (pos - lo)) + ordered[hi] * (pos - lo)


def _comma_ints(value: str) -> list[int]:
    return [int(item.strip()) for item in value.split(",") if item.strip()]


def resolve_lengths(args: argparse.Namespace, device: torch.device) -> torch.Tensor:
    """Per-request lengths: explicit ``--lengths`` or a pattern (microbench.py:90-130)."""

    if args.lengths:
        values = _comma_ints(args.lengths)
        if len(values) == 1:
            values = values * args.batch
        if len(values) != args.batch:
            raise ValueError("--lengths needs 1 or batch comma-separated values")
    else:
        pattern = args.length_pattern
        if pattern == "uniform":
            values = [args.seq_len] * args.batch
        elif pattern == "descending":
            lo = max(1, args.seq_len // 4)
            values = [args.seq_len] if args.batch == 1 else [
                int(round(args.seq_len - (args.seq_len - lo) * i / (args.batch - 1))) for i in range(args.batch)]
        elif pattern == "bimodal":
            short = max(1, args.seq_len // 4)
            split = args.batch // 2
            values = [args.seq_len] * split + [short] * (args.batch - split)
        elif pattern == "random":
            generator = torch.Generator(device="cpu")
            generator.manual_seed(int(args.seed))
            lo = max(1, args.seq_len // 4)
            values = torch.randint(lo, args.seq_len + 1, (args.batch,), generator=generator).tolist()
        else:
            raise ValueError("--length-pattern must be uniform, descending, bimodal or random")
    if any(v < 1 or v > args.seq_len for v in values):
        raise ValueError("effective lengths must lie in [1, seq_len]")
    return torch.tensor(values, dtype=torch.int64, device=device)


def measure_latency_ms(run: Callable[[], torch.Tensor], device: torch.device, warmup: int, repeats: int,
                       iters: int) -> tuple[torch.Tensor, list[float], str]:
    """Events around ``iters`` calls per repeat on GPU, perf_counter on CPU (microbench.py:133-179)."""

    out = run()
    for _ in range(max(0, warmup)):
        out = run()
    synchronize(device)
    raw: list[float] = []
    repeats, iters = max(1, repeats), max(1, iters)
    if device.type == "cuda":
        method = "cuda_event"
        for _ in range(repeats):
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record()
            for _ in range(iters):
                out = run()
            end.record()
            end.synchronize()
            raw.append(float(start.elapsed_time(end) / iters))
    else:
        method = "perf_counter"
        for _ in range(repeats):
            t0 = perf_counter()
            for _ in range(iters):
                out = run()
            raw.append(float((perf_counter() - t0) * 1000.0 / iters))
    synchronize(device)
    return out, raw, method


def measure_graph_latency_ms(run: Callable[[], torch.Tensor], iters: int, repeats: int) -> list[float]:
    """Per-call latency of ``iters`` calls captured into one HIP graph and replayed ``repeats`` times
    (events around each replay): the device time of the launch sequence without the host's per-call
    work.  The HIP backends' launches are capture-safe (the merged split plans zero-fill their own
    merge area inside the capture)."""

    iters, repeats = max(1, iters), max(1, repeats)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(iters):
            run()
    graph.replay()
    torch.cuda.synchronize()
    raw = []
    for _ in range(repeats):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        graph.replay()
        end.record()
        end.synchronize()
        raw.append(float(start.elapsed_time(end) / iters))
    return raw


def cli_args(args: argparse.Namespace, *, repeats: int = 1, json_flag: bool = True) -> list[str]:
    out = ["--backend", args.backend, "--batch", str(args.batch), "--heads", str(args.heads),
           "--seq-len", str(args.seq_len), "--head-dim", str(args.head_dim), "--block-size", str(args.block_size),
           "--iters", str(max(1, args.iters)), "--warmup", str(max(1, args.warmup)), "--repeats", str(repeats),
           "--device", "cuda", "--dtype", args.dtype, "--paged-layout", args.paged_layout,
           "--layout-seed", str(args.layout_seed), "--length-pattern", args.length_pattern, "--seed", str(args.seed)]
    if args.lengths:
        out += ["--lengths", args.lengths]
    if json_flag:
        out.append("--json")
    return out


def rocprof_commands(args: argparse.Namespace) -> dict[str, str]:
    bench = " ".join(["python", "-m", "flashspec_amd.microbench", *cli_args(args)])
    regex = KERNEL_REGEX.get(args.backend)
    filt = f" --kernel-include-regex '{regex}'" if regex else ""
    tag = f"{args.backend}_b{args.batch}_h{args.heads}_s{args.seq_len}_d{args.head_dim}"
    return {
        "kernel_trace": f"rocprofv3 --kernel-trace --stats -d results/rocprof_{tag} -o trace -- {bench}",
        "hbm_fetch": f"rocprofv3 --pmc FETCH_SIZE{filt} -d results/rocprof_{tag}_fetch -o fetch -- {bench}",
        "hbm_write": f"rocprofv3 --pmc WRITE_SIZE{filt} -d results/rocprof_{tag}_write -o write -- {bench}",
    }


def resource_row(backend: str, head_dim: int, dtype: torch.dtype) -> dict | None:
    """Compiler-reported registers/occupancy of the HIP kernel a backend launches."""

    path = Path(__file__).resolve().with_name("kernel_resources.json")
    if backend not in KERNEL_REGEX or not path.exists():
        return None
    paged = "Lb1" if backend == "triton_paged" else "Lb0"
    tname = {torch.float16: "6__half", torch.bfloat16: "14__hip_bfloat16", torch.float32: "f"}.get(dtype)
    want = f"decode_rows_kernelILi{head_dim}E{tname}{paged}E"
    for row in json.loads(path.read_text()).get("kernels", []):
        if want in row.get("kernel", ""):
            return row
    return None


def latency_breakdown(args, stats: dict, latency_ms: float, method: str) -> list[dict]:
    """Stage definitions with work estimates (microbench.py:312-403)."""

    elements = float(args.batch * args.heads * args.seq_len * args.head_dim)
    output_bytes = float(args.batch * args.heads * args.head_dim * 4)
    quant, dense = float(stats["quant_kv_bytes"]), float(stats["dense_kv_bytes"])
    portable = args.backend in {"fused", "paged"}
    accelerated = args.backend in {"triton_fused", "triton_paged"}
    kv_load = quant + dense if portable else (quant if accelerated else dense)
    materialized = dense if portable else 0.0
    dequant_ops = 4.0 * elements if args.backend != "dense" else 0.0
    softmax_ops = 3.0 * args.batch * args.heads * args.seq_len
    return [
        {"stage": "kv_load", "estimated_bytes": kv_load, "estimated_flops_or_ops": 0.0,
         "measurement": "rocprofv3 FETCH_SIZE", "notes": "K/V reads (int8 + scale/zero on the HIP path)"},
        {"stage": "dequant", "estimated_bytes": materialized, "estimated_flops_or_ops": dequant_ops,
         "measurement": "rocprofv3 SQ counters", "notes": "int8 -> fp32 with zero point and scale"},
        {"stage": "qk", "estimated_bytes": 0.0, "estimated_flops_or_ops": 2.0 * elements,
         "measurement": "rocprofv3 SQ counters", "notes": "score per cached token"},
        {"stage": "softmax", "estimated_bytes": 0.0, "estimated_flops_or_ops": softmax_ops,
         "measurement": "rocprofv3 SQ counters", "notes": "online max / exp / sum"},
        {"stage": "pv_accumulation", "estimated_bytes": 0.0, "estimated_flops_or_ops": 2.0 * elements,
         "measurement": "rocprofv3 SQ counters", "notes": "probability-weighted V sum"},
        {"stage": "output_write", "estimated_bytes": output_bytes, "estimated_flops_or_ops": 0.0,
         "measurement": "rocprofv3 WRITE_SIZE", "notes": "[batch, heads, head_dim] output"},
        {"stage": "total_kernel_or_backend", "estimated_bytes": kv_load + materialized + output_bytes,
         "estimated_flops_or_ops": 4.0 * elements + softmax_ops + dequant_ops, "measurement": method,
         "measured_latency_ms": latency_ms, "notes": "total from the benchmark timing"},
    ]


def _csv_rows(directory: str, suffix: str) -> list[dict]:
    import csv

    rows = []
    for path in glob.glob(os.path.join(directory, "**", f"*{suffix}"), recursive=True):
        with open(path, newline="") as fh:
            rows.extend(csv.DictReader(fh))
    return rows


def _profile(args, result: dict) -> None:
    """Run this benchmark under rocprofv3 (child processes, the program itself after ``--``) in
    three passes -- kernel trace, FETCH_SIZE, WRITE_SIZE -- and backfill the measured_* fields.

    Per step: the matching kernels' median durations and median per-dispatch bytes, summed over
    the distinct kernels a step launches (the decode, plus the split merge when rows split).
    FETCH_SIZE is scaled by FETCH_SIZE_SCALE (gfx950 counts half of the bytes a copy reads)."""

    import re

    regex = KERNEL_REGEX.get(args.backend)
    pat = re.compile(regex) if regex else None
    bench = [sys.executable, "-m", "flashspec_amd.microbench", *cli_args(args, json_flag=False)]
    env = dict(os.environ, TMPDIR=tempfile.gettempdir())
    with tempfile.TemporaryDirectory() as tmp:
        passes = {"trace": ["--kernel-trace"], "fetch": ["--pmc", "FETCH_SIZE"], "write": ["--pmc", "WRITE_SIZE"]}
        found = {}
        for name, opts in passes.items():
            cmd = [args.rocprof_bin, *opts, "--output-format", "csv"]
            if regex and name != "trace":
                cmd += ["--kernel-include-regex", regex]
            cmd += ["-d", os.path.join(tmp, name), "-o", name, "--", *bench]
            try:
                proc = subprocess.run(cmd, capture_output=True, text=True, timeout=args.profile_timeout,
                                      cwd=str(Path(__file__).resolve().parents[1]), env=env)
            except (FileNotFoundError, subprocess.TimeoutExpired) as exc:
                result["profiler_error"] = f"rocprofv3 {name} pass failed: {exc}"
                return
            suffix = "kernel_trace.csv" if name == "trace" else "counter_collection.csv"
            rows = _csv_rows(os.path.join(tmp, name), suffix)
            # rocprofv3 may exit non-zero after the program finished with whole results; only
            # missing output counts as a failure
            if not rows:
                result["profiler_error"] = f"rocprofv3 {name} exited {proc.returncode} without {suffix}: " \
                                           f"{proc.stderr[-600:]}"
                return
            found[name] = rows

        durations: dict[str, list[float]] = {}
        for r in found["trace"]:
            if pat is None or pat.search(r["Kernel_Name"]):
                durations.setdefault(r["Kernel_Name"], []).append(
                    (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e6)

        def per_dispatch(rows, counter):
            by_kernel: dict[str, dict[str, float]] = {}
            for r in rows:
                if r["Counter_Name"] == counter and (pat is None or pat.search(r["Kernel_Name"])):
                    d = by_kernel.setdefault(r["Kernel_Name"], {})
                    d[r["Dispatch_Id"]] = d.get(r["Dispatch_Id"], 0.0) + float(r["Counter_Value"])
            return {k: statistics.median(v.values()) for k, v in by_kernel.items()}

        fetch = per_dispatch(found["fetch"], "FETCH_SIZE")
        write = per_dispatch(found["write"], "WRITE_SIZE")
        if not durations or not fetch:
            result["profiler_warning"] = "no matching kernels in the rocprofv3 output"
            return
        dur_ms = sum(statistics.median(v) for v in durations.values())
        fetched = sum(fetch.values()) * 1024 * FETCH_SIZE_SCALE
        written = sum(write.values()) * 1024
        result.update({
            "bandwidth_fields_are_estimates": False,
            "measured_dram_bytes": fetched + written,
            "measured_achieved_bandwidth_gbps": (fetched + written) / (dur_ms * 1e-3) / 1e9,
            "measured_dram_throughput_pct": 100.0 * (fetched + written) / (dur_ms * 1e-3) / 1e9 / PEAK_HBM_GBPS,
            "measured_kernel_duration_ms": dur_ms,
            "measured_kernel_count": sum(len(v) for v in durations.values()),
            "measured_kernel_names": sorted(durations),
            "profiler_metrics_source": "rocprofv3",
        })


def parse_args(argv=None) -> argparse.Namespace:
    p = argparse.ArgumentParser(description="flashspec_amd decode attention microbenchmark")
    p.add_argument("--batch", type=int, default=4)
    p.add_argument("--heads", type=int, default=8)
    p.add_argument("--seq-len", type=int, default=512)
    p.add_argument("--head-dim", type=int, default=64)
    p.add_argument("--block-size", type=int, default=16)
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--lengths", default="")
    p.add_argument("--length-pattern", default="uniform", choices=["uniform", "descending", "bimodal", "random"])
    p.add_argument("--paged-layout", default="contiguous", choices=["contiguous", "shuffled", "interleaved"])
    p.add_argument("--layout-seed", type=int, default=0)
    p.add_argument("--iters", type=int, default=10)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--repeats", type=int, default=10)
    p.add_argument("--backend", choices=["dense", "fused", "triton_fused", "paged", "triton_paged"], default="paged")
    p.add_argument("--device", default="auto")
    p.add_argument("--dtype", default="auto", choices=DTYPE_CHOICES)
    p.add_argument("--json", action="store_true")
    p.add_argument("--output", type=Path)
    p.add_argument("--raw-output", type=Path)
    p.add_argument("--include-raw", action="store_true")
    p.add_argument("--save-output", type=Path, help="write the attention output as a float32 .npy file")
    p.add_argument("--no-graph", action="store_true",
                   help="skip the graph-captured latency of the HIP backends (graph_latency_ms)")
    p.add_argument("--profile-rocprof", action="store_true", help="backfill measured_* fields with rocprofv3")
    p.add_argument("--rocprof-bin", default="rocprofv3")
    p.add_argument("--profile-timeout", type=float, default=600.0)
    return p.parse_args(argv)


def main(argv=None) -> dict:
    args = parse_args(argv)
    device = resolve_device(args.device)
    dtype = resolve_dtype(args.dtype, device)
    generator = torch.Generator(device=device)
    generator.manual_seed(args.seed)
    q = torch.randn((args.batch, args.heads, args.head_dim), generator=generator, device=device, dtype=dtype)
    k = torch.randn((args.batch, args.heads, args.seq_len, args.head_dim), generator=generator, device=device,
                    dtype=dtype)
    v = torch.randn((args.batch, args.heads, args.seq_len, args.head_dim), generator=generator, device=device,
                    dtype=dtype)
    lengths = resolve_lengths(args, device)
    attention_lengths = None if args.length_pattern == "uniform" and not args.lengths else lengths

    if args.backend == "dense":
        def run():
            return reference_attention(q, k, v, lengths=attention_lengths)

        nbytes = float(2 * k.numel() * k.element_size())
        stats = {"dense_kv_bytes": nbytes, "quant_kv_bytes": nbytes, "compression_ratio": 1.0,
                 "materializes_dense_kv": 0.0}
    elif args.backend in ("fused", "triton_fused"):
        if args.backend == "triton_fused" and (not HAS_TRITON or device.type != "cuda"):
            raise RuntimeError("triton_fused needs the HIP library and a GPU device")
        kq = quantize_int8_per_block(k, block_size=args.block_size)
        vq = quantize_int8_per_block(v, block_size=args.block_size)
        fn = fused_dequant_attention_triton if args.backend == "triton_fused" else fused_dequant_attention

        def run():
            return fn(q, kq, vq, lengths=attention_lengths)

        _, stats = fn(q, kq, vq, lengths=attention_lengths, return_stats=True)
    else:
        if args.backend == "triton_paged" and (not HAS_TRITON or device.type != "cuda"):
            raise RuntimeError("triton_paged needs the HIP library and a GPU device")
        cache = PagedKVCache.from_dense(k, v, block_size=args.block_size, lengths=attention_lengths,
                                        block_table_pattern=args.paged_layout, layout_seed=args.layout_seed)
        fn = paged_quant_attention_triton if args.backend == "triton_paged" else paged_quant_attention

        def run():
            return fn(q, cache)

        _, stats = fn(q, cache, return_stats=True)
    if args.backend != "dense":
        del k, v  # the quantized copies are what the timed closures read

    out, raw, method = measure_latency_ms(run, device, args.warmup, args.repeats, args.iters)
    latency = statistics.median(raw)
    denom = max(1.0e-9, latency / 1000.0)
    dense_bw = stats["dense_kv_bytes"] / denom / 1.0e9
    quant_bw = stats["quant_kv_bytes"] / denom / 1.0e9
    res = resource_row(args.backend, args.head_dim, dtype)
    commands = rocprof_commands(args)
    result = {
        "backend": args.backend, "device": str(device), "device_name": device_name(device),
        "dtype": str(dtype).replace("torch.", ""), "batch": args.batch, "heads": args.heads,
        "seq_len": args.seq_len, "head_dim": args.head_dim, "block_size": args.block_size, "seed": args.seed,
        "length_pattern": args.length_pattern, "passes_lengths_to_attention": attention_lengths is not None,
        "effective_lengths": [int(x) for x in lengths.cpu().tolist()],
        "effective_min_seq_len": int(lengths.min().item()), "effective_max_seq_len": int(lengths.max().item()),
        "paged_layout": args.paged_layout, "paged_layout_seed": args.layout_seed,
        "iters": args.iters, "warmup": args.warmup, "repeats": args.repeats, "timing_method": method,
        "latency_ms": latency, "latency_mean_ms": statistics.fmean(raw),
        "latency_std_ms": statistics.pstdev(raw) if len(raw) > 1 else 0.0,
        "latency_min_ms": min(raw), "latency_max_ms": max(raw),
        "latency_p50_ms": _percentile(raw, 50.0), "latency_p90_ms": _percentile(raw, 90.0),
        "latency_p99_ms": _percentile(raw, 99.0),
        "tokens_per_second": args.batch / denom,
        "estimated_dense_kv_bytes": stats["dense_kv_bytes"], "estimated_quant_kv_bytes": stats["quant_kv_bytes"],
        "compression_ratio": stats["compression_ratio"],
        "materializes_dense_kv": bool(stats["materializes_dense_kv"]),
        "num_splits": stats.get("num_splits"), "block_n": stats.get("block_n"), "num_warps": stats.get("num_warps"),
        "env_flashspec_num_splits": os.environ.get("FLASHSPEC_NUM_SPLITS"),
        "env_flashspec_block_n": os.environ.get("FLASHSPEC_BLOCK_N"),
        "env_flashspec_num_warps": os.environ.get("FLASHSPEC_NUM_WARPS"),
        "bandwidth_fields_are_estimates": True,
        "estimated_effective_dense_kv_bandwidth_gbps": dense_bw,
        "estimated_effective_quant_kv_bandwidth_gbps": quant_bw,
        "effective_dense_kv_bandwidth_gbps": dense_bw, "effective_quant_kv_bandwidth_gbps": quant_bw,
        "measured_kernel_latency_ms": latency if method == "cuda_event" else None,
        "measured_latency_p50_ms": _percentile(raw, 50.0), "measured_latency_p90_ms": _percentile(raw, 90.0),
        "measured_latency_p99_ms": _percentile(raw, 99.0),
        "measured_dram_bytes": None, "measured_achieved_bandwidth_gbps": None, "measured_occupancy_pct": None,
        "measured_sm_utilization_pct": None, "measured_dram_throughput_pct": None,
        "measured_registers_per_thread": None if res is None else res.get("vgprs"),
        "measured_theoretical_occupancy_pct": None if res is None else 100.0 * res.get("occupancy", 0) / 8.0,
        "registers_source": None if res is None else "compiler kernel-resource-usage for gfx950",
        "measured_kernel_duration_ms": None, "measured_kernel_count": None, "measured_kernel_names": None,
        "profiler_metrics_source": "rocprofv3_required_for_dram_bytes",
        "nsight_compute_command": commands["hbm_fetch"],
        "nsight_compute_source_command": commands["kernel_trace"],
        "nsight_compute_commands": {"metrics_csv": commands["hbm_fetch"],
                                    "source_instruction_report": commands["kernel_trace"]},
        "rocprof_commands": commands,
        "latency_breakdown": latency_breakdown(args, stats, latency, method),
        "output_checksum": float(out.float().sum().item()),
    }
    if args.backend.startswith("triton_") and device.type == "cuda" and not args.no_graph:
        graph_raw = measure_graph_latency_ms(run, args.iters, args.repeats)
        result["graph_latency_ms"] = statistics.median(graph_raw)
        result["graph_latency_note"] = (f"{args.iters} calls captured in one HIP graph, median of {args.repeats} "
                                        "replays, per call")
    if args.save_output:
        args.save_output.parent.mkdir(parents=True, exist_ok=True)
        np.save(args.save_output, out.detach().float().cpu().numpy())
    if args.include_raw:
        result["raw_latency_ms"] = raw
    if args.profile_rocprof:
        if device.type != "cuda":
            result["profiler_error"] = "--profile-rocprof needs a GPU device"
        else:
            _profile(args, result)
    if args.output:
        args.output.parent.mkdir(parents=True, exist_ok=True)
        args.output.write_text(json.dumps(result, indent=2), encoding="utf-8")
    if args.raw_output:
        args.raw_output.parent.mkdir(parents=True, exist_ok=True)
        args.raw_output.write_text(json.dumps({"raw_latency_ms": raw}, indent=2), encoding="utf-8")
    if args.json:
        print(json.dumps(result, indent=2))
    else:
        for key, value in result.items():
            print(f"{key}: {value}")
    return result


if __name__ == "__main__":
    main()
