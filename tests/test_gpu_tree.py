"""GPU parity of tree verification (fs_tree_verify_i8) against the oracle (oracle/tree.py).

Attention within max-abs 2e-3 / max-rel 1e-2 (fp16 outputs).  Cases cover chains (which
reduce to paged decode over prefix + path), stars, random forests, empty prefixes, the
shuffled page layout, 8-token and per-token quantization, head dims 64/96/128/256, and the
prefix partials of rows that split.
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

import flashspec_amd as fa
from flashspec_amd import _lib
from oracle import tree as ot
from tests._helpers import assert_attention_close, from_cache, np_of, randn

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)


def announce(msg: str) -> None:
    print(f"[gpu case] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(autouse=True)
def _require_gpu(monkeypatch):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    assert _lib.available(), _lib.LOAD_ERROR
    for key in ("FLASHSPEC_NUM_SPLITS", "FLASHSPEC_BLOCK_N", "FLASHSPEC_NUM_WARPS"):
        monkeypatch.delenv(key, raising=False)


def _random_parents(B, N, seed):
    rng = np.random.default_rng(seed)
    par = np.full((B, N), -1, dtype=np.int64)
    for b in range(B):
        for n in range(1, N):
            par[b, n] = rng.integers(-1, n)
    return par


def _run(B, H, S, D, N, parents, lengths, page=16, layout="shuffled", q_dtype=torch.float16, kv_format="affine_block",
         seed=0):
    q = randn((B, N, H, D), seed + 1, q_dtype)
    k = randn((B, H, S, D), seed + 2)
    v = randn((B, H, S, D), seed + 3)
    dk = randn((B, N, H, D), seed + 4)
    dv = randn((B, N, H, D), seed + 5)
    cache = fa.PagedKVCache.from_dense(k.to(DEV), v.to(DEV), page, lengths=torch.tensor(lengths).to(DEV),
                                       block_table_pattern=layout, layout_seed=seed, kv_format=kv_format)
    got, stats = fa.tree_verify_attention(q.to(DEV), cache, dk.to(DEV), dv.to(DEV),
                                          torch.tensor(parents).to(DEV), return_stats=True)
    torch.cuda.synchronize(DEV)
    ref = ot.tree_verify_attention(np_of(q.float()), from_cache(cache), np_of(dk.float()), np_of(dv.float()),
                                   np.asarray(parents))
    return got, ref, stats


@pytest.mark.parametrize("B,H,S,D,N,kind,lengths", [
    (2, 4, 300, 128, 6, "chain", [300, 77]),
    (2, 4, 300, 128, 6, "star", [300, 77]),
    (3, 8, 513, 128, 8, "random", [513, 1, 200]),
    (2, 2, 129, 64, 5, "random", [129, 0]),        # an empty prefix
    (1, 4, 700, 256, 4, "random", [700]),
    (2, 3, 90, 96, 7, "random", [90, 45]),
])
def test_tree_verify_matches_oracle(B, H, S, D, N, kind, lengths):
    announce(f"tree verify B{B} H{H} S{S} D{D} N{N} {kind} lengths={lengths}")
    if kind == "chain":
        parents = np.tile(np.arange(-1, N - 1), (B, 1))
    elif kind == "star":
        parents = np.full((B, N), -1)
    else:
        parents = _random_parents(B, N, S + N)
    got, ref, stats = _run(B, H, S, D, N, parents, lengths, seed=B + S)
    assert stats["materializes_dense_kv"] == 0.0
    assert_attention_close(got.reshape(B * N, H, D), ref.reshape(B * N, H, D), torch.float16, f"tree {kind}")


@pytest.mark.parametrize("page,kv_format,q_dtype", [(8, "affine_block", torch.float16),
                                                    (16, "symmetric_token", torch.bfloat16),
                                                    (32, "affine_block", torch.float32)])
def test_tree_verify_formats(page, kv_format, q_dtype):
    announce(f"tree verify page{page} {kv_format} {q_dtype}")
    B, H, S, D, N = 2, 4, 260, 128, 6
    parents = _random_parents(B, N, page)
    got, ref, _ = _run(B, H, S, D, N, parents, [260, 100], page=page, kv_format=kv_format, q_dtype=q_dtype)
    assert_attention_close(got.reshape(B * N, H, D), ref.reshape(B * N, H, D), q_dtype, kv_format)


def test_tree_verify_split_rows(monkeypatch):
    """Prefix rows that split (forced 4 splits) merge their partials in the tail kernel."""

    announce("tree verify with forced split-K")
    monkeypatch.setenv("FLASHSPEC_NUM_SPLITS", "4")
    B, H, S, D, N = 1, 2, 2048, 128, 5
    parents = np.array([[-1, 0, 1, 0, 3]])
    got, ref, stats = _run(B, H, S, D, N, parents, [2048], seed=9)
    assert stats["num_splits"] == 4.0
    assert_attention_close(got.reshape(B * N, H, D), ref.reshape(B * N, H, D), torch.float16, "split")


def test_tree_single_node_matches_paged_decode_plus_token():
    """One root node: the tree output equals paged decode over the prefix extended by the
    node's own token, computed by the oracle as plain attention over concatenated K/V."""

    announce("tree verify single node")
    B, H, S, D = 2, 4, 200, 128
    got, ref, _ = _run(B, H, S, D, 1, np.full((B, 1), -1), [200, 64], seed=21)
    assert_attention_close(got.reshape(B, H, D), ref.reshape(B, H, D), torch.float16, "single node")
