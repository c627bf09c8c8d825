"""GPU parity of the per-channel affine INT8 KV format (oracle quant.quantize_int8_per_channel):
quantize and page store bit-exact, fused and paged decode within max-abs 2e-3 / max-rel 1e-2
(tiled kernel at head_dim 64/128/256 with 16/32/64-token blocks, the element-wise kernel for
8-token blocks and head_dim 40, split-K, ragged lengths, the three page layouts).
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

import flashspec_amd as fa
from flashspec_amd import _lib
from oracle import attention as oa
from oracle import paged as op
from oracle import quant as oq
from tests._helpers import assert_attention_close, assert_quant_equal, from_cache, from_qt, np_of, randn, to_qt

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


def sync():
    torch.cuda.synchronize(DEV)


def _channel_scaled(shape, seed, dtype=torch.float16):
    """randn with per-channel magnitudes spread over 2 decades, largest ~3 (the case per-channel
    scales serve; outputs stay O(1), where the 2e-3 absolute tolerance is above fp16's ulp)."""

    g = torch.Generator().manual_seed(seed)
    mag = 10.0 ** (torch.rand(shape[-1], generator=g) * 2 - 1.5)
    return (torch.randn(shape, generator=g) * mag).to(dtype)


@pytest.mark.parametrize("shape,bs,dtype", [((2, 4, 100, 128), 16, torch.float16), ((3, 2, 64, 64), 32, torch.float32),
                                            ((1, 3, 37, 24), 8, torch.bfloat16)])
def test_quantize_per_channel_bit_exact(shape, bs, dtype):
    announce(f"quantize per-channel {shape} bs{bs} {dtype}")
    x = _channel_scaled(shape, sum(shape), dtype)
    got = fa.quantize_int8_per_channel(x.to(DEV), bs)
    sync()
    ref = oq.quantize_int8_per_channel(np_of(x.float()), bs)
    assert_quant_equal(from_qt(got), ref, "per-channel quantize")
    back = fa.dequantize_int8_per_block(got)
    sync()
    assert np.array_equal(np_of(back), oq.dequantize_int8_per_block(ref))


@pytest.mark.parametrize("layout", ["contiguous", "shuffled", "interleaved"])
def test_from_dense_per_channel_pages_bit_exact(layout):
    announce(f"from_dense per-channel layout={layout}")
    k, v = _channel_scaled((3, 4, 70, 64), 31), _channel_scaled((3, 4, 70, 64), 32)
    lengths = torch.tensor([70, 33, 1])
    cache = fa.PagedKVCache.from_dense(k.to(DEV), v.to(DEV), block_size=16, lengths=lengths.to(DEV),
                                       block_table_pattern=layout, layout_seed=3, kv_format="affine_channel")
    sync()
    table = np_of(cache.block_table)
    perm = None
    if layout != "contiguous":
        perm = np.empty(table.size, dtype=np.int64)
        perm[table.ravel()] = np.arange(table.size)
    ref = op.from_dense(np_of(k.float()), np_of(v.float()), 16, lengths=np_of(lengths), perm=perm,
                        kv_format="affine_channel")
    assert_quant_equal(from_qt(cache.k_quant), ref.k_quant, "k")
    assert_quant_equal(from_qt(cache.v_quant), ref.v_quant, "v")


@pytest.mark.parametrize("B,H,S,D,bs,q_dtype,lengths,tiled", [
    (2, 4, 300, 128, 16, torch.float16, None, True),
    (2, 4, 300, 128, 64, torch.bfloat16, [300, 17], True),
    (3, 2, 257, 64, 32, torch.float32, [257, 0, 100], True),
    (2, 4, 500, 128, 48, torch.float16, [500, 97], True),      # 3 tiles per block
    (1, 4, 2000, 64, 128, torch.float16, [1990], True),        # 8 tiles per block, ragged last block
    (1, 4, 700, 256, 16, torch.float16, None, True),
    (2, 3, 90, 96, 16, torch.float16, [90, 45], True),
    (2, 3, 90, 128, 8, torch.float16, [90, 45], False),   # 8-token blocks: element-wise kernel
    (2, 2, 77, 40, 16, torch.float16, [77, 5], False),     # head_dim 40: element-wise kernel
])
def test_fused_per_channel_matches_oracle(B, H, S, D, bs, q_dtype, lengths, tiled):
    announce(f"fused per-channel B{B} H{H} S{S} D{D} bs{bs} {q_dtype} lengths={lengths}")
    seed = B * 100 + S + bs
    q = randn((B, H, D), seed, q_dtype)
    kq = oq.quantize_int8_per_channel(np_of(_channel_scaled((B, H, S, D), seed + 1).float()), bs)
    vq = oq.quantize_int8_per_channel(np_of(_channel_scaled((B, H, S, D), seed + 2).float()), bs)
    lens = None if lengths is None else torch.tensor(lengths, dtype=torch.int64)
    got, stats = fa.fused_dequant_attention_triton(q.to(DEV), to_qt(kq, DEV), to_qt(vq, DEV),
                                                   lengths=None if lens is None else lens.to(DEV), return_stats=True)
    sync()
    assert stats["tiled_path"] == float(tiled)
    ref = oa.fused_dequant_attention(np_of(q.float()), kq, vq, None if lens is None else lens.numpy())
    if lengths is not None and 0 in lengths:
        keep = [i for i, L in enumerate(lengths) if L != 0]
        got, ref = got[keep], ref[keep]
    assert_attention_close(got, ref, q_dtype, "fused per-channel")


@pytest.mark.parametrize("layout,page,q_dtype", [("contiguous", 16, torch.float16), ("shuffled", 32, torch.bfloat16),
                                                 ("interleaved", 64, torch.float32)])
def test_paged_per_channel_matches_oracle(layout, page, q_dtype):
    announce(f"paged per-channel {layout} page{page} {q_dtype}")
    B, H, S, D = 3, 4, 300, 128
    q = randn((B, H, D), 41 + page, q_dtype)
    k, v = _channel_scaled((B, H, S, D), 42 + page), _channel_scaled((B, H, S, D), 43 + page)
    lens = torch.tensor([300, 31, 16], dtype=torch.int64)
    cache = fa.PagedKVCache.from_dense(k.to(DEV), v.to(DEV), block_size=page, lengths=lens.to(DEV),
                                       block_table_pattern=layout, layout_seed=5, kv_format="affine_channel")
    got, stats = fa.paged_quant_attention_triton(q.to(DEV), cache, return_stats=True)
    sync()
    assert stats["tiled_path"] == 1.0 and stats["num_warps"] <= 8.0
    ref = oa.paged_quant_attention(np_of(q.float()), from_cache(cache))
    assert_attention_close(got, ref, q_dtype, "paged per-channel")


def test_paged_per_channel_split_k(monkeypatch):
    announce("paged per-channel split-K")
    B, H, S, D = 2, 4, 2048, 128
    q = randn((B, H, D), 51)
    k, v = _channel_scaled((B, H, S, D), 52), _channel_scaled((B, H, S, D), 53)
    cache = fa.PagedKVCache.from_dense(k.to(DEV), v.to(DEV), block_size=16, kv_format="affine_channel")
    monkeypatch.setenv("FLASHSPEC_NUM_SPLITS", "4")
    got, st = fa.paged_quant_attention_triton(q.to(DEV), cache, return_stats=True)
    sync()
    assert st["num_splits"] == 4.0
    ref = oa.paged_quant_attention(np_of(q.float()), from_cache(cache))
    assert_attention_close(got, ref, torch.float16, "per-channel split")


@pytest.mark.parametrize("splits", ["1", "3"])
def test_paged_per_channel_whole_block_waves(monkeypatch, splits):
    """64-token blocks: waves take whole blocks of 4 tiles; splits of whole blocks, ragged rows."""
    announce(f"paged per-channel page64 splits={splits}")
    B, H, S, D = 3, 4, 2048, 128
    q = randn((B, H, D), 61)
    k, v = _channel_scaled((B, H, S, D), 62), _channel_scaled((B, H, S, D), 63)
    lens = torch.tensor([2048, 1000, 77], dtype=torch.int64)
    cache = fa.PagedKVCache.from_dense(k.to(DEV), v.to(DEV), block_size=64, lengths=lens.to(DEV),
                                       block_table_pattern="shuffled", layout_seed=9, kv_format="affine_channel")
    monkeypatch.setenv("FLASHSPEC_NUM_SPLITS", splits)
    got, st = fa.paged_quant_attention_triton(q.to(DEV), cache, return_stats=True)
    sync()
    assert st["tiled_path"] == 1.0 and st["num_splits"] == float(splits)
    ref = oa.paged_quant_attention(np_of(q.float()), from_cache(cache))
    assert_attention_close(got, ref, torch.float16, "per-channel whole-block waves")
