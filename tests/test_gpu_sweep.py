"""Seeded randomized parity sweeps of paged and fused decode and of tree verification against the CPU oracle.

Each case draws batch, heads, head_dim, page size, KV format, query dtype, page layout and
ragged lengths (empty and one-token rows included) from its own seed, so the hand-picked
parity cases' kernel paths also meet in combinations nobody listed: the 64/128/256-dim
layouts, head_dims that are multiples of 4 but not of 16 (the straddling lane) or not
multiples of 4 (generic kernel), sub-tile pages, per-token / FP8 / per-channel parameters (single-tile and
whole-block waves), forced split counts.  Attention within max-abs 2e-3 / max-rel 1e-2 of
the oracle, zero rows for empty requests.
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

import flashspec_amd as fa
from flashspec_amd import _lib
from oracle import attention as oa
from tests._helpers import assert_attention_close, from_cache, np_of, randn

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)
HEAD_DIMS = (16, 20, 24, 32, 34, 36, 40, 44, 48, 64, 72, 96, 100, 104, 120, 128, 136, 160, 200, 212, 248, 256)
PAGES = (8, 16, 32, 48, 64)
FORMATS = ("affine_block", "symmetric_token", "fp8_block", "affine_channel")
QDTYPES = (torch.float16, torch.bfloat16, torch.float32)
LAYOUTS = ("contiguous", "shuffled", "interleaved")


@pytest.fixture(autouse=True)
def _require_gpu(monkeypatch):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    assert _lib.available(), _lib.LOAD_ERROR
    for key in ("FLASHSPEC_NUM_SPLITS", "FLASHSPEC_BLOCK_N", "FLASHSPEC_NUM_WARPS", "FLASHSPEC_TREE_NODES_PER_WG"):
        monkeypatch.delenv(key, raising=False)


def _draw(seed: int) -> dict:
    r = np.random.default_rng(1000 + seed)
    B, H = int(r.integers(1, 4)), int(r.integers(1, 5))
    S = int(r.integers(1, 700))
    lengths = [int(r.choice([S, r.integers(0, S + 1), 1, 0], p=[0.4, 0.4, 0.1, 0.1])) for _ in range(B)]
    lengths[0] = S  # max_seq_len stays S
    return dict(B=B, H=H, S=S, D=int(r.choice(HEAD_DIMS)), page=int(r.choice(PAGES)), fmt=str(r.choice(FORMATS)),
                q_dtype=QDTYPES[int(r.integers(0, 3))], layout=str(r.choice(LAYOUTS)), lengths=lengths,
                splits=[None, "1", "3"][int(r.integers(0, 3))])


@pytest.mark.parametrize("seed", range(80))
def test_paged_decode_random_sweep(monkeypatch, seed):
    c = _draw(seed)
    print(f"[gpu case] sweep seed={seed} {c}", flush=True)
    sys.stdout.flush()
    if c["splits"] is not None:
        monkeypatch.setenv("FLASHSPEC_NUM_SPLITS", c["splits"])
        monkeypatch.setenv("FLASHSPEC_BLOCK_N", "16")
    B, H, S, D = c["B"], c["H"], c["S"], c["D"]
    q = randn((B, H, D), 7 * seed + 1, c["q_dtype"])
    k, v = randn((B, H, S, D), 7 * seed + 2), randn((B, H, S, D), 7 * seed + 3)
    lens = torch.tensor(c["lengths"], dtype=torch.int64)
    cache = fa.PagedKVCache.from_dense(k.to(DEV), v.to(DEV), block_size=c["page"], lengths=lens.to(DEV),
                                       block_table_pattern=c["layout"], layout_seed=seed, kv_format=c["fmt"])
    got = fa.paged_quant_attention_triton(q.to(DEV), cache)
    torch.cuda.synchronize(DEV)
    ref = oa.paged_quant_attention(np_of(q.float()), from_cache(cache))
    keep = [i for i, L in enumerate(c["lengths"]) if L > 0]
    empty = [i for i, L in enumerate(c["lengths"]) if L == 0]
    if empty:
        assert (got[empty] == 0).all(), "empty rows must be zero"
    assert_attention_close(got[keep], ref[keep], c["q_dtype"], f"sweep seed {seed}")


def _quantize(x: torch.Tensor, fmt: str, block: int):
    if fmt == "affine_block":
        return fa.quantize_int8_per_block(x, block)
    if fmt == "fp8_block":
        return fa.quantize_fp8_per_block(x, block)
    if fmt == "affine_channel":
        return fa.quantize_int8_per_channel(x, block)
    return fa.quantize_int8_symmetric_per_token(x)


@pytest.mark.parametrize("seed", range(40))
def test_fused_decode_random_sweep(monkeypatch, seed):
    c = _draw(500 + seed)
    print(f"[gpu case] fused sweep seed={seed} {c}", flush=True)
    sys.stdout.flush()
    if c["splits"] is not None:
        monkeypatch.setenv("FLASHSPEC_NUM_SPLITS", c["splits"])
        monkeypatch.setenv("FLASHSPEC_BLOCK_N", "16")
    B, H, S, D = c["B"], c["H"], c["S"], c["D"]
    q = randn((B, H, D), 11 * seed + 1, c["q_dtype"])
    k, v = randn((B, H, S, D), 11 * seed + 2).to(DEV), randn((B, H, S, D), 11 * seed + 3).to(DEV)
    kq, vq = _quantize(k, c["fmt"], c["page"]), _quantize(v, c["fmt"], c["page"])
    lens = torch.tensor(c["lengths"], dtype=torch.int64)
    got = fa.fused_dequant_attention_triton(q.to(DEV), kq, vq, lengths=lens.to(DEV))
    torch.cuda.synchronize(DEV)
    from tests._helpers import from_qt
    ref = oa.fused_dequant_attention(np_of(q.float()), from_qt(kq), from_qt(vq), lens.numpy())
    keep = [i for i, L in enumerate(c["lengths"]) if L > 0]
    empty = [i for i, L in enumerate(c["lengths"]) if L == 0]
    if empty:
        assert (got[empty] == 0).all(), "empty rows must be zero"
    assert_attention_close(got[keep], ref[keep], c["q_dtype"], f"fused sweep seed {seed}")


def _draw_tree(seed: int) -> dict:
    r = np.random.default_rng(7000 + seed)
    B, H = int(r.integers(1, 4)), int(r.integers(1, 5))
    S = int(r.integers(1, 500))
    lengths = [S] + [int(r.integers(0, S + 1)) for _ in range(B - 1)]
    N = int(r.choice([1, 3, 16, 17, 31, 33, 48, 64, 70]))
    parents = np.full((B, N), -1, dtype=np.int64)
    for n in range(1, N):
        parents[:, n] = r.integers(-1, n, size=B)
    return dict(B=B, H=H, S=S, D=int(r.choice((64, 96, 128, 256))), N=N, page=int(r.choice((16, 32, 64))),
                fmt=str(r.choice(FORMATS)), q_dtype=QDTYPES[int(r.integers(0, 3))], lengths=lengths,
                parents=parents, kernel=str(r.choice(("auto", "rows"))), per_wg=[None, "32"][int(r.integers(0, 2))],
                splits=[None, "1", "3"][int(r.integers(0, 3))])


@pytest.mark.parametrize("seed", range(30))
def test_tree_verify_random_sweep(monkeypatch, seed):
    from oracle import tree as ot

    c = _draw_tree(seed)
    print(f"[gpu case] tree sweep seed={seed} { {k: v for k, v in c.items() if k != 'parents'} }", flush=True)
    sys.stdout.flush()
    if c["splits"] is not None:
        monkeypatch.setenv("FLASHSPEC_NUM_SPLITS", c["splits"])
        monkeypatch.setenv("FLASHSPEC_BLOCK_N", "16")
    if c["per_wg"] is not None:
        monkeypatch.setenv("FLASHSPEC_TREE_NODES_PER_WG", c["per_wg"])
    B, H, S, D, N = c["B"], c["H"], c["S"], c["D"], c["N"]
    q = randn((B, N, H, D), 13 * seed + 1, c["q_dtype"])
    k, v = randn((B, H, S, D), 13 * seed + 2), randn((B, H, S, D), 13 * seed + 3)
    dk = randn((B, N, H, D), 13 * seed + 4, torch.float32).to(c["q_dtype"])
    dv = randn((B, N, H, D), 13 * seed + 5, torch.float32).to(c["q_dtype"])
    cache = fa.PagedKVCache.from_dense(k.to(DEV), v.to(DEV), block_size=c["page"],
                                       lengths=torch.tensor(c["lengths"]).to(DEV), block_table_pattern="shuffled",
                                       layout_seed=seed, kv_format=c["fmt"])
    got = fa.tree_verify_attention(q.to(DEV), cache, dk.to(DEV), dv.to(DEV), torch.tensor(c["parents"]),
                                   kernel=c["kernel"])
    torch.cuda.synchronize(DEV)
    ref = ot.tree_verify_attention(np_of(q.float()), from_cache(cache), np_of(dk.float()), np_of(dv.float()),
                                   c["parents"])
    assert_attention_close(got.reshape(B * N, H, D), ref.reshape(B * N, H, D), c["q_dtype"], f"tree sweep {seed}")
