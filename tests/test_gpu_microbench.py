"""The microbench CLI's HIP backends on the GPU (restates reference benchmarks/microbench.py:444-631
and the schema test tests/test_flashspec.py:263-324), each run as ``python -m
flashspec_amd.microbench`` in a fresh child process; plus one ``--profile-rocprof`` run whose
rocprofv3 passes (kernel trace, FETCH_SIZE, WRITE_SIZE; reference microbench.py:262-309 used Nsight
Compute) backfill the measured_* fields."""

from __future__ import annotations

import json
import math
import os
import shutil
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import paged as op
from oracle import quant as oq
from tests._helpers import assert_attention_close

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]

SCHEMA_KEYS = ("backend", "seq_len", "head_dim", "block_size", "num_splits", "block_n", "env_flashspec_num_splits",
               "env_flashspec_block_n", "env_flashspec_num_warps", "num_warps", "length_pattern",
               "passes_lengths_to_attention", "effective_lengths", "effective_min_seq_len", "effective_max_seq_len",
               "paged_layout", "paged_layout_seed", "bandwidth_fields_are_estimates",
               "measured_registers_per_thread", "measured_theoretical_occupancy_pct",
               "nsight_compute_source_command", "nsight_compute_commands", "materializes_dense_kv")


def _microbench(*args: str, timeout: float = 240) -> dict:
    env = os.environ.copy()
    for knob in ("FLASHSPEC_NUM_SPLITS", "FLASHSPEC_BLOCK_N", "FLASHSPEC_NUM_WARPS"):
        env.pop(knob, None)
    cmd = [sys.executable, "-m", "flashspec_amd.microbench", "--device", "cuda", "--dtype", "float16", "--json",
           *args]
    print("microbench:", " ".join(args), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True, env=env, cwd=ROOT, timeout=timeout)
    assert proc.returncode == 0, proc.stderr[-3000:]
    return json.loads(proc.stdout)


def _check_hip_result(data: dict, backend: str, batch: int, seq_len: int) -> None:
    for key in SCHEMA_KEYS:
        assert key in data, key
    assert data["backend"] == backend and data["device"].startswith("cuda")
    assert data["materializes_dense_kv"] is False
    assert data["timing_method"] == "cuda_event"
    assert math.isfinite(data["latency_ms"]) and data["latency_ms"] > 0
    assert math.isfinite(data["output_checksum"])
    assert data["effective_lengths"] == [seq_len] * batch
    # the HIP launch plan is reported: 16-token tiles knob (block_n), waves per workgroup, splits
    assert data["block_n"] == 128.0 and data["num_warps"] in (1.0, 2.0, 4.0, 8.0, 16.0)
    assert data["num_splits"] >= 1.0
    assert data["measured_registers_per_thread"] is not None


@pytest.mark.parametrize("layout", ["contiguous", "shuffled"])
def test_microbench_triton_paged_backend(layout):
    """Config C3's shape through the paged HIP kernel, both page layouts."""

    data = _microbench("--backend", "triton_paged", "--batch", "8", "--heads", "32", "--seq-len", "2048",
                       "--head-dim", "128", "--paged-layout", layout, "--iters", "20", "--warmup", "5",
                       "--repeats", "5")
    _check_hip_result(data, "triton_paged", 8, 2048)
    assert data["paged_layout"] == layout
    # int8 K/V + fp32 scale + int16 zero per 16-token page and head, + int64 table and lengths
    assert data["estimated_quant_kv_bytes"] == 2 * (8 * 32 * 2048 * 128 + 8 * 32 * 128 * 6) + 8 * 128 * 8 + 8 * 8


def test_microbench_triton_fused_backend_c1():
    """Config C1 (B4 H32 S2048 D128) through the contiguous HIP kernel."""

    data = _microbench("--backend", "triton_fused", "--batch", "4", "--heads", "32", "--seq-len", "2048",
                       "--head-dim", "128", "--iters", "20", "--warmup", "5", "--repeats", "5")
    _check_hip_result(data, "triton_fused", 4, 2048)
    # the graph-captured latency (no per-call host work) beside the eager one
    assert math.isfinite(data["graph_latency_ms"]) and 0 < data["graph_latency_ms"] < 1.0
    print(f"C1 eager {data['latency_ms'] * 1e3:.2f} us, graph {data['graph_latency_ms'] * 1e3:.2f} us", flush=True)


@pytest.mark.parametrize("backend", ["triton_paged", "triton_fused"])
def test_microbench_hip_output_matches_the_oracle(backend, tmp_path):
    """The CLI's HIP backends, element-wise against the CPU oracle on the same seeded inputs
    (descending lengths, B2 H4 S300 D64): the child process saves its output (--save-output), this
    process draws the same q, k, v from the same seeded device generator (microbench.py's draw
    order) and runs the oracle's quantizer and attention on them."""

    path = tmp_path / "out.npy"
    data = _microbench("--backend", backend, "--batch", "2", "--heads", "4", "--seq-len", "300", "--head-dim", "64",
                       "--iters", "2", "--warmup", "1", "--repeats", "2", "--length-pattern", "descending",
                       "--save-output", str(path))
    assert data["materializes_dense_kv"] is False
    assert data["graph_latency_ms"] > 0
    out = np.load(path, allow_pickle=False)
    dev = torch.device("cuda", 0)
    g = torch.Generator(device=dev)
    g.manual_seed(0)
    q = torch.randn((2, 4, 64), generator=g, device=dev, dtype=torch.float16)
    k = torch.randn((2, 4, 300, 64), generator=g, device=dev, dtype=torch.float16)
    v = torch.randn((2, 4, 300, 64), generator=g, device=dev, dtype=torch.float16)
    lengths = np.array(data["effective_lengths"], dtype=np.int64)
    kf, vf, qf = (t.float().cpu().numpy() for t in (k, v, q))
    if backend == "triton_paged":
        ref = oa.paged_quant_attention(qf, op.from_dense(kf, vf, 16, lengths=lengths))
    else:
        ref = oa.fused_dequant_attention(qf, oq.quantize_int8_per_block(kf, 16), oq.quantize_int8_per_block(vf, 16),
                                         lengths)
    assert_attention_close(torch.from_numpy(out).to(torch.float16), ref, torch.float16, backend)


@pytest.mark.timeout(600)
def test_microbench_profile_rocprof_backfills_measured_fields():
    """--profile-rocprof at config C3: rocprofv3 runs the benchmark three times (trace, FETCH_SIZE,
    WRITE_SIZE) and the measured HBM bytes land within 0.95-1.10 of the algorithmic bytes."""

    if shutil.which("rocprofv3") is None:
        pytest.skip("rocprofv3 not on PATH")
    data = _microbench("--backend", "triton_paged", "--batch", "8", "--heads", "32", "--seq-len", "2048",
                       "--head-dim", "128", "--iters", "10", "--warmup", "3", "--repeats", "3",
                       "--profile-rocprof", "--profile-timeout", "150", timeout=560)
    assert "profiler_error" not in data, data.get("profiler_error")
    assert "profiler_warning" not in data, data.get("profiler_warning")
    assert data["bandwidth_fields_are_estimates"] is False
    assert data["profiler_metrics_source"] == "rocprofv3"
    assert any("decode_rows_kernel" in n for n in data["measured_kernel_names"])
    algorithmic = data["estimated_quant_kv_bytes"] + 2 * 8 * 32 * 128 * 2  # + fp16 q and output
    ratio = data["measured_dram_bytes"] / algorithmic
    print(f"measured / algorithmic bytes = {ratio:.4f}, kernel {data['measured_kernel_duration_ms'] * 1e3:.2f} us",
          flush=True)
    assert 0.95 <= ratio <= 1.10
    assert 0 < data["measured_kernel_duration_ms"] < 1.0
    assert 0 < data["measured_dram_throughput_pct"] <= 100.0
