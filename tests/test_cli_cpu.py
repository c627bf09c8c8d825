"""CLI JSON schemas of the microbench and serving entry points, run as subprocesses on CPU.

Restates reference tests/test_flashspec.py:263-324 (microbench keys and defaults) and
:326-378 (serving latency and allocator keys) against ``python -m flashspec_amd.microbench``
and ``python -m flashspec_amd.serving``.
"""

from __future__ import annotations

import json
import os
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def _run_module(module: str, *args: str) -> dict:
    env = os.environ.copy()
    for knob in ("FLASHSPEC_NUM_SPLITS", "FLASHSPEC_BLOCK_N", "FLASHSPEC_NUM_WARPS"):
        env.pop(knob, None)
    proc = subprocess.run([sys.executable, "-m", module, *args], check=True, capture_output=True, text=True,
                          env=env, cwd=ROOT, timeout=300)
    return json.loads(proc.stdout)


def test_microbench_json_schema_includes_experiment_knobs():
    data = _run_module("flashspec_amd.microbench", "--backend", "dense", "--batch", "1", "--heads", "1",
                       "--seq-len", "4", "--head-dim", "8", "--iters", "1", "--warmup", "0", "--repeats", "1",
                       "--device", "cpu", "--dtype", "float32", "--json")
    for key in ("backend", "seq_len", "head_dim", "block_size", "num_splits", "block_n", "env_flashspec_num_splits",
                "env_flashspec_block_n", "env_flashspec_num_warps", "num_warps", "length_pattern",
                "passes_lengths_to_attention", "effective_lengths", "effective_min_seq_len",
                "effective_max_seq_len", "paged_layout", "paged_layout_seed", "bandwidth_fields_are_estimates",
                "measured_registers_per_thread", "measured_theoretical_occupancy_pct",
                "nsight_compute_source_command", "nsight_compute_commands", "materializes_dense_kv"):
        assert key in data, key
    assert data["block_n"] is None
    assert data["num_warps"] is None
    assert data["env_flashspec_num_splits"] is None
    assert data["env_flashspec_block_n"] is None
    assert data["env_flashspec_num_warps"] is None
    assert data["length_pattern"] == "uniform"
    assert data["passes_lengths_to_attention"] is False
    assert data["effective_lengths"] == [4]
    assert data["paged_layout"] == "contiguous"


@pytest.mark.parametrize("pattern", ["descending", "random"])
def test_microbench_paged_length_patterns(pattern):
    """Descending runs from seq_len down to seq_len // 4; random draws from [seq_len // 4, seq_len]
    with a CPU generator seeded by --seed (microbench.py:107-126)."""

    data = _run_module("flashspec_amd.microbench", "--backend", "paged", "--batch", "4", "--heads", "2",
                       "--seq-len", "40", "--head-dim", "16", "--length-pattern", pattern, "--paged-layout",
                       "shuffled", "--iters", "1", "--warmup", "0", "--repeats", "1", "--device", "cpu",
                       "--dtype", "float32", "--json")
    if pattern == "descending":
        assert data["effective_lengths"] == [40, 30, 20, 10]
    else:
        assert all(10 <= n <= 40 for n in data["effective_lengths"])
    assert data["passes_lengths_to_attention"] is True
    assert data["paged_layout"] == "shuffled"
    assert data["materializes_dense_kv"] is True
    assert data["effective_max_seq_len"] == max(data["effective_lengths"])


def test_serving_json_schema_includes_latency_and_allocator_fields():
    data = _run_module("flashspec_amd.serving", "--requests", "2", "--prompt-lens", "3,5",
                       "--prompt-length-distribution", "bimodal", "--decode-steps", "3", "--request-life-steps",
                       "2", "--heads", "1", "--head-dim", "8", "--block-size", "4", "--device", "cpu", "--dtype",
                       "float32", "--json")
    for key in ("ttft_ms", "tpot_ms", "tokens_per_second", "prefill_ms", "decode_ms", "block_utilization",
                "fragmentation", "allocated_blocks", "free_blocks", "live_requests", "used_tokens",
                "capacity_tokens", "padding_waste", "arrivals", "finishes", "prompt_lens"):
        assert key in data, key
    assert data["prompt_lens"] == [3, 5]
    assert data["finishes"] >= 2
