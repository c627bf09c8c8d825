"""GPU parity of the FP8 E4M3 KV format (oracle/fp8.py): quantize / page store / dequantize
bit-exact, fused and paged decode attention within max-abs 2e-3 / max-rel 1e-2 of the oracle
(tiled kernel at head_dim 64/96/128/256 and quant blocks 16/32/8/1, the generic kernel at head_dim
40, split-K, ragged lengths, all three page layouts).
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

import flashspec_amd as fa
from flashspec_amd import _lib
from oracle import attention as oa
from oracle import fp8 as of
from oracle import paged as op
from tests._helpers import assert_attention_close, assert_quant_equal, from_cache, from_qt, np_of, randn

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


@pytest.mark.parametrize("shape,bs,dtype,scale", [((2, 4, 100, 128), 16, torch.float16, 1.0),
                                                  ((3, 2, 64, 64), 32, torch.float32, 1e-3),
                                                  ((1, 3, 37, 24), 8, torch.bfloat16, 200.0),
                                                  ((2, 2, 19, 128), 1, torch.float16, 1.0),
                                                  ((1, 1, 5, 40), 16, torch.float32, 1e-7)])
def test_quantize_fp8_bit_exact(shape, bs, dtype, scale):
    announce(f"quantize fp8 {shape} bs{bs} {dtype} x{scale}")
    x = (randn(shape, sum(shape) + bs, torch.float32) * scale).to(dtype)
    got = fa.quantize_fp8_per_block(x.to(DEV), bs)
    sync()
    ref = of.quantize_fp8_per_block(np_of(x.float()), bs)
    assert got.values.dtype == torch.float8_e4m3fn
    assert_quant_equal(from_qt(got), ref, "fp8 quantize")
    back = fa.dequantize_int8_per_block(got)
    sync()
    assert np.array_equal(np_of(back), of.dequantize_fp8_per_block(ref))


@pytest.mark.parametrize("layout", ["contiguous", "shuffled", "interleaved"])
def test_from_dense_fp8_pages_bit_exact(layout):
    announce(f"from_dense fp8 layout={layout}")
    k = randn((3, 4, 70, 64), 11)
    v = randn((3, 4, 70, 64), 12)
    lengths = torch.tensor([70, 33, 1])
    cache = fa.PagedKVCache.from_dense(k.to(DEV), v.to(DEV), block_size=16, lengths=lengths.to(DEV),
                                       block_table_pattern=layout, layout_seed=3, kv_format="fp8_block")
    sync()
    table = np_of(cache.block_table)
    perm = None
    if layout != "contiguous":
        perm = np.empty(table.size, dtype=np.int64)
        perm[table.ravel()] = np.arange(table.size)
    ref = op.from_dense(np_of(k.float()), np_of(v.float()), 16, lengths=np_of(lengths), perm=perm,
                        kv_format="fp8_block")
    assert_quant_equal(from_qt(cache.k_quant), ref.k_quant, "k")
    assert_quant_equal(from_qt(cache.v_quant), ref.v_quant, "v")


def _fused_fp8(B, H, S, D, bs, seed, q_dtype):
    q = randn((B, H, D), seed, q_dtype)
    k = randn((B, H, S, D), seed + 1)
    v = randn((B, H, S, D), seed + 2)
    return q, of.quantize_fp8_per_block(np_of(k.float()), bs), of.quantize_fp8_per_block(np_of(v.float()), bs)


@pytest.mark.parametrize("B,H,S,D,bs,q_dtype,lengths", [
    (2, 4, 300, 128, 16, torch.float16, None),
    (2, 4, 300, 128, 16, torch.bfloat16, [300, 17]),
    (3, 2, 257, 64, 32, torch.float32, [257, 0, 100]),
    (1, 4, 700, 256, 16, torch.float16, None),
    (2, 3, 90, 96, 8, torch.float16, [90, 45]),
    (2, 2, 77, 40, 16, torch.float16, [77, 5]),      # head_dim 40: an odd multiple of 8
    (2, 4, 160, 128, 1, torch.float16, [160, 33]),   # one scale per token
    (2, 2, 90, 56, 1, torch.bfloat16, [90, 41]),     # head_dim 56, one scale per token
    (2, 2, 70, 44, 16, torch.float16, [70, 9]),      # head_dim 44: 12 straddling dims
    (2, 2, 80, 148, 1, torch.bfloat16, [80, 21]),    # head_dim 148: 4 straddling dims, one scale per token
    (2, 2, 75, 100, 16, torch.bfloat16, [75, 18]),   # head_dim 100, bf16 q on the fp16 score path, block scales
    (2, 2, 70, 42, 16, torch.float16, [70, 9]),      # generic kernel: head_dim 42
])
def test_fused_fp8_matches_oracle(B, H, S, D, bs, q_dtype, lengths):
    from tests._helpers import to_qt

    announce(f"fused fp8 B{B} H{H} S{S} D{D} bs{bs} {q_dtype} lengths={lengths}")
    q, kq, vq = _fused_fp8(B, H, S, D, bs, B * 100 + S + bs, q_dtype)
    lens = None if lengths is None else torch.tensor(lengths, dtype=torch.int64)
    got, stats = fa.fused_dequant_attention_triton(q.to(DEV), to_qt(kq, DEV), to_qt(vq, DEV),
                                                   lengths=None if lens is None else lens.to(DEV), return_stats=True)
    sync()
    # tiled: head_dim a multiple of 16, or one of 4 from 20 on with block / per-token scales
    assert stats["tiled_path"] == float(D % 16 == 0 or (D % 4 == 0 and D >= 20 and (bs == 1 or bs % 16 == 0)))
    ref = oa.fused_dequant_attention(np_of(q.float()), kq, vq, None if lens is None else lens.numpy())
    if lengths is not None and 0 in lengths:
        keep = [i for i, L in enumerate(lengths) if L != 0]
        assert (got[[i for i, L in enumerate(lengths) if L == 0]] == 0).all()
        got, ref = got[keep], ref[keep]
    assert_attention_close(got, ref, q_dtype, "fused fp8")


@pytest.mark.parametrize("layout,page,q_dtype,D", [("contiguous", 16, torch.float16, 128),
                                                   ("shuffled", 16, torch.bfloat16, 128),
                                                   ("interleaved", 32, torch.float32, 128),
                                                   ("shuffled", 64, torch.float16, 128),
                                                   ("shuffled", 16, torch.bfloat16, 100),  # straddling lane
                                                   ("contiguous", 32, torch.float16, 36)])
def test_paged_fp8_matches_oracle(layout, page, q_dtype, D):
    announce(f"paged fp8 {layout} page{page} {q_dtype} D{D}")
    B, H, S = 3, 4, 300
    q = randn((B, H, D), 21 + page, q_dtype)
    k, v = randn((B, H, S, D), 22 + page), randn((B, H, S, D), 23 + page)
    lens = torch.tensor([300, 31, 16], dtype=torch.int64)
    cache = fa.PagedKVCache.from_dense(k.to(DEV), v.to(DEV), block_size=page, lengths=lens.to(DEV),
                                       block_table_pattern=layout, layout_seed=5, kv_format="fp8_block")
    got, stats = fa.paged_quant_attention_triton(q.to(DEV), cache, return_stats=True)
    sync()
    assert stats["materializes_dense_kv"] == 0.0 and stats["tiled_path"] == 1.0
    ref = oa.paged_quant_attention(np_of(q.float()), from_cache(cache))
    assert_attention_close(got, ref, q_dtype, "paged fp8")


def test_paged_fp8_split_k_and_metric_shape(monkeypatch):
    """The metric shape (B8 H32 S4096 D128, 16-token pages) in FP8 against the oracle, and a
    forced 4-way split-K against the single-split result."""

    announce("paged fp8 metric shape + split-K")
    B, H, S, D = 8, 32, 4096, 128
    g = torch.Generator().manual_seed(0)
    q = torch.randn((B, H, D), generator=g).to(torch.float16)
    k = torch.randn((B, H, S, D), generator=g).to(torch.float16)
    v = torch.randn((B, H, S, D), generator=g).to(torch.float16)
    cache = fa.PagedKVCache.from_dense(k.to(DEV), v.to(DEV), block_size=16, kv_format="fp8_block")
    got = fa.paged_quant_attention_triton(q.to(DEV), cache)
    monkeypatch.setenv("FLASHSPEC_NUM_SPLITS", "4")
    split, st = fa.paged_quant_attention_triton(q.to(DEV), cache, return_stats=True)
    sync()
    assert st["num_splits"] == 4.0
    assert float((got.float() - split.float()).abs().max()) <= 2e-3
    sel = [0, 5]
    ref = oa.paged_quant_attention(np_of(q[sel].float()), op.OracleCache(
        from_qt(cache.k_quant), from_qt(cache.v_quant), np_of(cache.block_table)[sel].astype(np.int64),
        np_of(cache.lengths)[sel].astype(np.int64), 16, S))
    assert_attention_close(got[sel], ref, torch.float16, "metric fp8")


def test_fp8_cache_rejected_where_unsupported():
    k = randn((1, 2, 32, 64), 1).to(DEV)
    cache = fa.PagedKVCache.from_dense(k, k, 16, kv_format="fp8_block")
    with pytest.raises(ValueError):
        cache.append(k[:, :, :1], k[:, :, :1])
