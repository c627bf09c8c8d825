"""GPU parity: the HIP kernels (through the public API and the C ABI) against the CPU oracle.

Integer/byte outputs (quantized values, scales, zero points, tables) must be
bit-exact; attention outputs must be within max-abs 2e-3 / max-rel 1e-2 (fp16).
Inputs are drawn on the CPU from seeded generators so they are device-independent.
"""

from __future__ import annotations

import os
import sys

import numpy as np
import pytest
import torch

import flashspec_amd as fa
from flashspec_amd import _lib, triton_utils
from oracle import attention as oa
from oracle import paged as op
from oracle import quant as oq
from tests._helpers import (
    assert_attention_close,
    assert_quant_equal,
    cast_like_q,
    from_cache,
    from_qt,
    golden_cache,
    golden_quant,
    load_npz,
    np_of,
    oracle_fused_attention,
    oracle_paged_attention,
    randn,
    to_cache,
    to_qt,
)

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


# ---- quantize / dequantize -------------------------------------------------------------------

def test_quantize_matches_reference_golden_vectors_bit_exact():
    d = load_npz("quant_golden.npz")
    for name in d["names"]:
        x = torch.from_numpy(d[f"{name}_x"]).to(DEV)
        bs = int(d[f"{name}_block"])
        announce(f"quantize golden {name} shape={tuple(x.shape)} bs={bs}")
        q = fa.quantize_int8_per_block(x, block_size=bs)
        sync()
        assert q.original_shape == tuple(x.shape)
        assert_quant_equal(from_qt(q), golden_quant(d, name), name)
        deq = fa.dequantize_int8_per_block(q)
        assert np.array_equal(np_of(deq).view(np.uint32), d[f"{name}_deq"].view(np.uint32)), name


@pytest.mark.parametrize("shape,bs,dtype", [
    ((2, 3, 19, 16), 8, torch.float32),
    ((8, 32, 300, 128), 16, torch.float16),
    ((2, 4, 50, 64), 16, torch.bfloat16),
    ((3, 1, 16, 256), 32, torch.float16),
    ((5, 7, 24), 4, torch.float32),
    ((2, 3, 40, 32), 16, torch.float32),
    ((1, 2, 33, 256), 16, torch.float32),
    ((2, 2, 20, 128), 32, torch.bfloat16),
])
def test_quantize_bit_exact_against_oracle(shape, bs, dtype):
    announce(f"quantize shape={shape} bs={bs} dtype={dtype}")
    x = randn(shape, seed=sum(shape), dtype=dtype) * 3.0
    q = fa.quantize_int8_per_block(x.to(DEV), block_size=bs)
    ref = oq.quantize_int8_per_block(np_of(x.to(torch.float32)), bs)
    sync()
    assert_quant_equal(from_qt(q), ref, str(shape))
    out = fa.dequantize_int8_per_block(q)
    assert np.array_equal(np_of(out).view(np.uint32), oq.dequantize_int8_per_block(ref).view(np.uint32))
    half = fa.dequantize_int8_per_block(q, dtype=torch.float16)
    assert half.dtype == torch.float16
    assert torch.equal(half.cpu(), torch.from_numpy(oq.dequantize_int8_per_block(ref)).to(torch.float16))


def test_quantize_unaligned_source_bit_exact():
    """A source pointer that is not 16-byte aligned takes the element-wise kernel."""

    announce("quantize via C ABI from a 2-byte-offset fp16 source")
    S, D, bs = 37, 128, 16
    base = randn((2 * S * D + 1,), seed=5)
    x = base[1:].reshape(2, S, D)
    xd = base.to(DEV)
    nb = -(-S // bs)
    values = torch.empty((2, nb, bs, D), dtype=torch.int8, device=DEV)
    scale = torch.empty((2, nb), dtype=torch.float32, device=DEV)
    zero = torch.empty((2, nb), dtype=torch.int16, device=DEV)
    lib = _lib.require()
    _lib.check(lib.fs_quantize_i8(xd.data_ptr() + 2, _lib.dtype_code(torch.float16), 2, S, D, bs, values.data_ptr(),
                                  scale.data_ptr(), zero.data_ptr(), _lib.stream_ptr(DEV)))
    sync()
    ref = oq.quantize_int8_per_block(np_of(x.float()), bs)
    assert np.array_equal(np_of(values), ref.values)
    assert np.array_equal(np_of(scale).view(np.uint32), ref.scale.reshape(2, nb).view(np.uint32))
    assert np.array_equal(np_of(zero), ref.zero_point.reshape(2, nb))


@pytest.mark.parametrize("shape,dtype", [
    ((2, 4, 37, 128), torch.float16),
    ((3, 50, 64), torch.bfloat16),
    ((2, 2, 33, 96), torch.float32),     # 12 lanes per row: the one-wave-per-row kernel
    ((1, 1, 7, 256), torch.float16),
    ((2, 3, 19, 40), torch.float16),
])
def test_symmetric_per_token_quantize_bit_exact(shape, dtype):
    announce(f"symmetric per-token quantize shape={shape} dtype={dtype}")
    x = randn(shape, seed=sum(shape) + 1, dtype=dtype) * 4.0
    q = fa.quantize_int8_symmetric_per_token(x.to(DEV))
    ref = oq.quantize_int8_symmetric_per_token(np_of(x.to(torch.float32)))
    sync()
    assert_quant_equal(from_qt(q), ref, str(shape))
    assert q.block_size == 1


def _sym_fused_case(B, H, S, D, seed, q_dtype):
    q = randn((B, H, D), seed, q_dtype)
    k = randn((B, H, S, D), seed + 1)
    v = randn((B, H, S, D), seed + 2)
    return q, k, v


@pytest.mark.parametrize("B,H,S,D,q_dtype,lengths", [
    (2, 4, 129, 128, torch.float16, [129, 100]),      # ragged last tile of a contiguous row
    (4, 32, 2048, 128, torch.float16, None),          # config 1 shape
    (2, 2, 77, 64, torch.bfloat16, [77, 5]),
    (1, 2, 300, 256, torch.float16, None),
    (2, 3, 50, 96, torch.float32, [50, 17]),
    (2, 3, 120, 104, torch.float16, [120, 64]),     # head_dim 104: the straddling lane in token mode
    (2, 2, 90, 52, torch.bfloat16, [90, 33]),       # head_dim 52: 4 straddling dims in token mode
    (1, 3, 140, 124, torch.float32, None),          # head_dim 124: 12 straddling dims in token mode
])
def test_fused_symmetric_per_token_matches_oracle(B, H, S, D, q_dtype, lengths):
    announce(f"fused symmetric per-token B{B} H{H} S{S} D{D} {q_dtype} lengths={lengths}")
    q, k, v = _sym_fused_case(B, H, S, D, B * 7 + S, q_dtype)
    kq = fa.quantize_int8_symmetric_per_token(k.to(DEV))
    vq = fa.quantize_int8_symmetric_per_token(v.to(DEV))
    lens = None if lengths is None else torch.tensor(lengths, dtype=torch.int64)
    got, stats = fa.fused_dequant_attention_triton(q.to(DEV), kq, vq, lengths=None if lens is None else lens.to(DEV),
                                                   return_stats=True)
    sync()
    assert stats["tiled_path"] == 1.0
    rk = oq.quantize_int8_symmetric_per_token(np_of(k.float()))
    rv = oq.quantize_int8_symmetric_per_token(np_of(v.float()))
    ref = oa.fused_dequant_attention(np_of(q.float()), rk, rv, None if lens is None else np_of(lens))
    assert_attention_close(got, ref, q_dtype, "fused symmetric")


@pytest.mark.parametrize("layout,page", [("contiguous", 16), ("shuffled", 16), ("interleaved", 32)])
def test_paged_symmetric_per_token_matches_oracle(layout, page):
    announce(f"paged symmetric per-token {layout} page{page}")
    B, H, S, D = 3, 4, 300, 128
    q, k, v = _sym_fused_case(B, H, S, D, 40 + page, torch.float16)
    lens = torch.tensor([300, 31, 16], dtype=torch.int64)
    cache = fa.PagedKVCache.from_dense(k.to(DEV), v.to(DEV), block_size=page, lengths=lens.to(DEV),
                                       block_table_pattern=layout, layout_seed=5, kv_format="symmetric_token")
    got, stats = fa.paged_quant_attention_triton(q.to(DEV), cache, return_stats=True)
    sync()
    assert stats["tiled_path"] == 1.0
    assert_attention_close(got, oracle_paged_attention(q, cache), torch.float16, "paged symmetric")
    rk = oq.quantize_int8_symmetric_per_token(np_of(k.float()))
    rv = oq.quantize_int8_symmetric_per_token(np_of(v.float()))
    ref = oa.fused_dequant_attention(np_of(q.float()), rk, rv, np_of(lens))
    assert_attention_close(got, ref, torch.float16, "paged symmetric vs contiguous oracle")


def test_config2_symmetric_per_token_split_k(monkeypatch):
    """B8 H32 S4096 D128, symmetric per-token INT8, num_splits=4 with the fp32 LSE merge;
    rows of two requests checked against the oracle."""

    announce("config 2 symmetric per-token split-K B8 H32 S4096 D128")
    monkeypatch.setenv("FLASHSPEC_NUM_SPLITS", "4")
    B, H, S, D = 8, 32, 4096, 128
    g = torch.Generator(device=DEV)
    g.manual_seed(4)
    q = torch.randn((B, H, D), generator=g, device=DEV, dtype=torch.float16)
    k = torch.randn((B, H, S, D), generator=g, device=DEV, dtype=torch.float16)
    v = torch.randn((B, H, S, D), generator=g, device=DEV, dtype=torch.float16)
    kq, vq = fa.quantize_int8_symmetric_per_token(k), fa.quantize_int8_symmetric_per_token(v)
    got, stats = fa.fused_dequant_attention_triton(q, kq, vq, return_stats=True)
    sync()
    assert stats["num_splits"] == 4.0
    for b in (0, 5):
        rk = oq.quantize_int8_symmetric_per_token(np_of(k[b:b + 1].float()))
        rv = oq.quantize_int8_symmetric_per_token(np_of(v[b:b + 1].float()))
        ref = oa.fused_dequant_attention(np_of(q[b:b + 1].float()), rk, rv, None)
        assert_attention_close(got[b:b + 1], ref, torch.float16, f"request {b}")


def test_config2_affine_per_block_split_k(monkeypatch):
    """Config C2 in the reference's own format: B8 H32 S4096 D128, affine per-block INT8 (16-token
    blocks, quantized by the HIP quantizer and checked bit-exact against the oracle quantizer on the
    sampled requests), num_splits=4 with the fp32 LSE merge (reference triton_fused.py:697-744 and
    its split test tests/test_flashspec.py:107-125); rows of two requests against the oracle."""

    announce("config 2 affine per-block split-K B8 H32 S4096 D128")
    monkeypatch.setenv("FLASHSPEC_NUM_SPLITS", "4")
    B, H, S, D = 8, 32, 4096, 128
    g = torch.Generator(device=DEV)
    g.manual_seed(6)
    q = torch.randn((B, H, D), generator=g, device=DEV, dtype=torch.float16)
    k = torch.randn((B, H, S, D), generator=g, device=DEV, dtype=torch.float16)
    v = torch.randn((B, H, S, D), generator=g, device=DEV, dtype=torch.float16)
    kq, vq = fa.quantize_int8_per_block(k, 16), fa.quantize_int8_per_block(v, 16)
    got, stats = fa.fused_dequant_attention_triton(q, kq, vq, return_stats=True)
    sync()
    assert stats["num_splits"] == 4.0 and stats["materializes_dense_kv"] == 0.0
    for b in (1, 6):
        rk = oq.quantize_int8_per_block(np_of(k[b:b + 1].float()), 16)
        rv = oq.quantize_int8_per_block(np_of(v[b:b + 1].float()), 16)
        for name, ours, ref in (("K", kq, rk), ("V", vq, rv)):
            assert np.array_equal(ours.values[b:b + 1].cpu().numpy(), ref.values), f"{name} values request {b}"
            assert np.array_equal(ours.scale[b:b + 1].cpu().numpy().view(np.uint32),
                                  np.asarray(ref.scale, np.float32).view(np.uint32)), f"{name} scales request {b}"
            assert np.array_equal(ours.zero_point[b:b + 1].cpu().numpy(), ref.zero_point), f"{name} zeros {b}"
        ref = oa.fused_dequant_attention(np_of(q[b:b + 1].float()), rk, rv, None)
        assert_attention_close(got[b:b + 1], ref, torch.float16, f"request {b}")
    # the split plan agrees with one split on the whole batch
    monkeypatch.setenv("FLASHSPEC_NUM_SPLITS", "1")
    one = fa.fused_dequant_attention_triton(q, kq, vq)
    sync()
    assert (got.float() - one.float()).abs().max().item() <= 2e-3


# ---- paged cache construction, append, allocator ----------------------------------------------

@pytest.mark.parametrize("layout", ["contiguous", "shuffled", "interleaved"])
def test_from_dense_pages_bit_exact(layout):
    announce(f"from_dense layout={layout}")
    k = randn((3, 4, 70, 64), 1)
    v = randn((3, 4, 70, 64), 2)
    lengths = torch.tensor([70, 33, 1])
    cache = fa.PagedKVCache.from_dense(k.to(DEV), v.to(DEV), block_size=16, lengths=lengths.to(DEV),
                                       block_table_pattern=layout, layout_seed=3)
    sync()
    table = np_of(cache.block_table)
    perm = None
    if layout != "contiguous":
        perm = np.empty(table.size, dtype=np.int64)
        perm[table.ravel()] = np.arange(table.size)
    ref = op.from_dense(np_of(k.float()), np_of(v.float()), 16, lengths=np_of(lengths), perm=perm)
    assert np.array_equal(table, ref.block_table)
    assert_quant_equal(from_qt(cache.k_quant), ref.k_quant, "k")
    assert_quant_equal(from_qt(cache.v_quant), ref.v_quant, "v")
    kd, vd = cache.to_dense()
    rk, rv = op.to_dense(ref)
    assert np.array_equal(np_of(kd), rk) and np.array_equal(np_of(vd), rv)


def test_append_matches_reference_golden_vectors_bit_exact():
    d = load_npz("append_golden.npz")
    for name in d["names"]:
        announce(f"append golden {name}")
        cin = to_cache(golden_cache(d, f"{name}_in"), DEV)
        ref = golden_cache(d, f"{name}_out")
        out = cin.append(torch.from_numpy(d[f"{name}_kn"]).to(DEV), torch.from_numpy(d[f"{name}_vn"]).to(DEV))
        sync()
        assert np.array_equal(np_of(out.block_table), ref.block_table), name
        assert np.array_equal(np_of(out.lengths), ref.lengths), name
        assert out.max_seq_len == ref.max_seq_len
        assert_quant_equal(from_qt(out.k_quant), ref.k_quant, f"{name}/k")
        assert_quant_equal(from_qt(out.v_quant), ref.v_quant, f"{name}/v")


def test_append_fp16_tokens_bit_exact_against_oracle():
    announce("append fp16 B4 H8 D128 page16 T=21")
    k, v = randn((4, 8, 40, 128), 5), randn((4, 8, 40, 128), 6)
    kn, vn = randn((4, 8, 21, 128), 7), randn((4, 8, 21, 128), 8)
    lengths = torch.tensor([40, 17, 16, 0])
    cache = fa.PagedKVCache.from_dense(k.to(DEV), v.to(DEV), 16, lengths=lengths.to(DEV),
                                       block_table_pattern="shuffled", layout_seed=1)
    out = cache.append(kn.to(DEV), vn.to(DEV))
    sync()
    ref = op.append(from_cache(cache), np_of(kn.float()), np_of(vn.float()))
    assert np.array_equal(np_of(out.block_table), ref.block_table)
    assert_quant_equal(from_qt(out.k_quant), ref.k_quant, "k")
    assert_quant_equal(from_qt(out.v_quant), ref.v_quant, "v")
    q = randn((4, 8, 128), 9)
    announce("append fp16 -> paged attention")
    got = fa.paged_quant_attention_triton(q.to(DEV), out)
    assert_attention_close(got, oa.paged_quant_attention(np_of(q), ref), torch.float16, "after append")


def test_allocator_lifecycle_matches_reference_golden_vectors_bit_exact():
    d = load_npz("allocator_golden.npz")
    H, D, bs, cap = (int(x) for x in d["config"])
    alloc = fa.PagedKVAllocator(capacity_blocks=cap, heads=H, head_dim=D, block_size=bs, device=DEV)
    for step, (code, rid, n) in enumerate(d["script"]):
        announce(f"allocator golden step {step} op={code} rid={rid} n={n}")
        if code == 0:
            alloc.add_request(int(rid), torch.from_numpy(d[f"s{step}_k"]).to(DEV),
                              torch.from_numpy(d[f"s{step}_v"]).to(DEV))
        elif code == 1:
            alloc.append_request(int(rid), torch.from_numpy(d[f"s{step}_k"]).to(DEV),
                                 torch.from_numpy(d[f"s{step}_v"]).to(DEV))
        else:
            alloc.release_request(int(rid))
        sync()
        for t, key in ((alloc.k_quant, "k"), (alloc.v_quant, "v")):
            assert np.array_equal(np_of(t.values), d[f"s{step}_{key}values"]), (step, key)
            assert np.array_equal(np_of(t.scale).view(np.uint32), d[f"s{step}_{key}scale"].view(np.uint32))
            assert np.array_equal(np_of(t.zero_point), d[f"s{step}_{key}zero"])
        live = alloc.live_request_ids
        if live:
            c = alloc.to_cache(live)
            assert np.array_equal(np_of(c.block_table), d[f"s{step}_table"])


def test_allocator_batched_append_bit_exact_against_oracle():
    announce("allocator batched append H4 D64 page16")
    H, D, bs = 4, 64, 16
    alloc = fa.PagedKVAllocator(capacity_blocks=64, heads=H, head_dim=D, block_size=bs, device=DEV)
    ora = op.OracleAllocator(64, H, D, bs)
    lens = [5, 16, 31, 1]
    for rid, L in enumerate(lens):
        k, v = randn((1, H, L, D), 100 + rid), randn((1, H, L, D), 200 + rid)
        alloc.add_request(rid, k.to(DEV), v.to(DEV))
        ora.add_request(rid, np_of(k.float()), np_of(v.float()))
    alloc.release_request(1)
    ora.release_request(1)
    rids = [0, 2, 3]
    for step in range(20):
        kn, vn = randn((3, H, 1, D), 300 + step), randn((3, H, 1, D), 400 + step)
        alloc.append_batch(rids, kn.to(DEV), vn.to(DEV))
        ora.append_batch(rids, np_of(kn.float()), np_of(vn.float()))
    sync()
    assert np.array_equal(np_of(alloc.k_quant.values), ora.k_quant.values)
    assert np.array_equal(np_of(alloc.v_quant.scale).view(np.uint32), ora.v_quant.scale.view(np.uint32))
    q = randn((3, H, D), 77)
    cache = alloc.to_cache(rids)
    announce("allocator cache -> paged attention")
    got = fa.paged_quant_attention_triton(q.to(DEV), cache)
    assert_attention_close(got, oa.paged_quant_attention(np_of(q), ora.to_cache(rids)), torch.float16, "alloc")


# ---- attention parity ------------------------------------------------------------------------

def _fused_case(B, H, S, D, bs, seed, q_dtype=torch.float16, lengths=None):
    q = randn((B, H, D), seed, q_dtype)
    k = randn((B, H, S, D), seed + 1, torch.float16)
    v = randn((B, H, S, D), seed + 2, torch.float16)
    kq = oq.quantize_int8_per_block(np_of(k.float()), bs)
    vq = oq.quantize_int8_per_block(np_of(v.float()), bs)
    lens = None if lengths is None else torch.tensor(lengths, dtype=torch.int64)
    return q, kq, vq, lens


@pytest.mark.parametrize("B,H,S,D,bs,q_dtype,lengths", [
    (2, 3, 129, 64, 16, torch.float16, [129, 113]),       # reference GPU test shape
    (2, 4, 1500, 128, 16, torch.float16, [1500, 977]),    # reference split-K test shape
    (4, 32, 2048, 128, 16, torch.float16, None),          # config 1
    (2, 8, 700, 128, 16, torch.bfloat16, [700, 1]),
    (2, 8, 300, 128, 16, torch.float32, [0, 300]),
    (1, 2, 517, 256, 16, torch.float16, None),
    (2, 2, 77, 32, 16, torch.float16, [77, 40]),          # head_dim 32 on the 64-dim layout
    (2, 4, 333, 96, 16, torch.float16, [333, 200]),       # head_dim 96 on the 128-dim layout
    (2, 2, 260, 192, 32, torch.bfloat16, [260, 31]),      # head_dim 192, quant block 32
    (2, 3, 130, 80, 64, torch.float32, None),             # head_dim 80, quant block 64
    (2, 3, 200, 64, 8, torch.float16, [200, 99]),         # 8-token quant blocks (sub-tiles), 64-dim layout
    (2, 4, 301, 128, 8, torch.float16, [301, 150]),       # 8-token quant blocks, 128-dim layout
    (1, 2, 90, 256, 24, torch.bfloat16, [90]),            # 24-token quant blocks, 256-dim layout
    (1, 2, 100, 40, 16, torch.float16, [100]),            # head_dim 40: an odd multiple of 8 (straddling lane)
    (2, 3, 333, 120, 16, torch.bfloat16, [333, 200]),     # head_dim 120 on the 128-dim layout
    (1, 2, 260, 248, 32, torch.float32, None),            # head_dim 248 on the 256-dim layout
    (2, 2, 1500, 88, 16, torch.float16, [1500, 700]),     # head_dim 88, split-K
    (2, 2, 90, 36, 16, torch.float16, [90, 31]),          # head_dim 36: the straddling lane keeps 4 dims
    (1, 2, 150, 100, 16, torch.bfloat16, [150]),          # head_dim 100: 4 dims past 96 on the 128-dim layout
    (2, 2, 130, 220, 32, torch.float32, [130, 47]),       # head_dim 220: 12 dims past 208 on the 256-dim layout
    (2, 2, 90, 34, 16, torch.float16, [90, 31]),          # generic path: head_dim 34
])
def test_fused_attention_matches_oracle(B, H, S, D, bs, q_dtype, lengths):
    announce(f"fused B{B} H{H} S{S} D{D} bs{bs} {q_dtype} lengths={lengths}")
    q, kq, vq, lens = _fused_case(B, H, S, D, bs, seed=B * 1000 + S, q_dtype=q_dtype, lengths=lengths)
    got, stats = fa.fused_dequant_attention_triton(
        q.to(DEV), to_qt(kq, DEV), to_qt(vq, DEV), lengths=None if lens is None else lens.to(DEV),
        return_stats=True)
    sync()
    assert stats["materializes_dense_kv"] == 0.0
    ref = oa.fused_dequant_attention(np_of(q), kq, vq, None if lens is None else lens.numpy())
    if lengths is not None and 0 in lengths:
        zero_rows = [i for i, L in enumerate(lengths) if L == 0]
        assert (got[zero_rows] == 0).all()  # an empty row writes zeros (triton_utils.py:181-186)
        keep = [i for i, L in enumerate(lengths) if L != 0]
        got, ref = got[keep], ref[keep]
    assert_attention_close(got, ref, q_dtype, "fused")


@pytest.mark.parametrize("D,q_dtype,fmt", [(128, torch.float16, "int8"), (128, torch.bfloat16, "int8"),
                                           (128, torch.float32, "int8"), (128, torch.bfloat16, "fp8"),
                                           (128, torch.float16, "fp8"), (64, torch.float16, "int8"),
                                           (100, torch.bfloat16, "int8")])
def test_queries_not_16_byte_aligned(D, q_dtype, fmt):
    """Queries that start one element past a 16-byte boundary load value by value instead of as
    16-byte words; paged and fused outputs equal the aligned queries' bit for bit and match the
    oracle."""

    announce(f"unaligned queries D{D} {q_dtype} {fmt}")
    B, H, S = 2, 4, 300
    q = randn((B, H, D), 71 + D, q_dtype).to(DEV)
    base = torch.zeros(B * H * D + 1, dtype=q_dtype, device=DEV)
    qu = base[1:].view(B, H, D)
    qu.copy_(q)
    assert qu.is_contiguous() and qu.data_ptr() % 16 != 0
    k, v = randn((B, H, S, D), 72).to(DEV), randn((B, H, S, D), 73).to(DEV)
    kv_format = "fp8_block" if fmt == "fp8" else "affine_block"
    cache = fa.PagedKVCache.from_dense(k, v, block_size=16, kv_format=kv_format)
    quantize = fa.quantize_fp8_per_block if fmt == "fp8" else fa.quantize_int8_per_block
    kq, vq = quantize(k, 16), quantize(v, 16)
    paged_a = fa.paged_quant_attention_triton(q, cache)
    paged_u = fa.paged_quant_attention_triton(qu, cache)
    fused_a = fa.fused_dequant_attention_triton(q, kq, vq)
    fused_u = fa.fused_dequant_attention_triton(qu, kq, vq)
    sync()
    assert torch.equal(paged_a, paged_u) and torch.equal(fused_a, fused_u)
    assert_attention_close(paged_u, oracle_paged_attention(q.cpu(), cache), q_dtype, "unaligned q, paged")
    assert_attention_close(fused_u, oracle_fused_attention(q.cpu(), kq, vq), q_dtype, "unaligned q, fused")


def test_fused_head_dim_64_default_plan_takes_eight_waves(monkeypatch):
    """Contiguous rows at head_dim 64 (B8 H32 S2048, one split) plan 8-wave workgroups; the result
    matches the oracle and a forced 16-wave plan."""

    announce("fused head_dim 64, default 8-wave plan")
    for key in ("FLASHSPEC_NUM_WARPS", "FLASHSPEC_NUM_SPLITS", "FLASHSPEC_BLOCK_N"):
        monkeypatch.delenv(key, raising=False)
    q, kq, vq, _ = _fused_case(8, 32, 2048, 64, 16, seed=64)
    args = (q.to(DEV), to_qt(kq, DEV), to_qt(vq, DEV))
    got, stats = fa.fused_dequant_attention_triton(*args, return_stats=True)
    sync()
    assert stats["num_warps"] == 8.0 and stats["num_splits"] == 1.0
    assert_attention_close(got, oa.fused_dequant_attention(np_of(q), kq, vq, None), torch.float16, "fused d64")
    monkeypatch.setenv("FLASHSPEC_NUM_WARPS", "16")
    other, stats16 = fa.fused_dequant_attention_triton(*args, return_stats=True)
    sync()
    assert stats16["num_warps"] == 16.0
    assert (got.float() - other.float()).abs().max().item() <= 2e-3


def test_fused_split_k_is_used_and_matches_single_split(monkeypatch):
    announce("fused split vs single split")
    q, kq, vq, _ = _fused_case(2, 4, 1500, 128, 16, seed=5)
    args = (q.to(DEV), to_qt(kq, DEV), to_qt(vq, DEV))
    multi, stats = fa.fused_dequant_attention_triton(*args, return_stats=True)
    assert stats["num_splits"] > 1.0
    monkeypatch.setenv("FLASHSPEC_NUM_SPLITS", "1")
    single, stats1 = fa.fused_dequant_attention_triton(*args, return_stats=True)
    sync()
    assert stats1["num_splits"] == 1.0
    assert (multi.float() - single.float()).abs().max().item() <= 2e-3


def _paged_case(B, H, S, D, page, seed, layout="contiguous", lengths=None, q_dtype=torch.float16):
    q = randn((B, H, D), seed, q_dtype)
    k = randn((B, H, S, D), seed + 1)
    v = randn((B, H, S, D), seed + 2)
    lens = None if lengths is None else torch.tensor(lengths, dtype=torch.int64)
    cache = fa.PagedKVCache.from_dense(k.to(DEV), v.to(DEV), block_size=page,
                                       lengths=None if lens is None else lens.to(DEV),
                                       block_table_pattern=layout, layout_seed=seed)
    return q, cache


@pytest.mark.parametrize("B,H,S,D,page,layout,lengths", [
    (2, 3, 129, 64, 16, "contiguous", [129, 113]),        # reference GPU test shape
    (8, 32, 2048, 128, 16, "contiguous", None),           # config 3
    (16, 32, 4096, 128, 16, "shuffled", [4096 - 256 * i for i in range(16)]),     # config 4
    (16, 32, 4096, 128, 16, "interleaved", [4096 - 256 * i - 7 for i in range(16)]),  # config 4, ragged tails
    (3, 4, 300, 128, 32, "shuffled", [300, 17, 0]),       # two tiles per page
    (2, 2, 64, 256, 16, "interleaved", [64, 63]),
    (2, 2, 7, 64, 4, "contiguous", None),                 # generic path: page 4
    (2, 3, 50, 48, 16, "shuffled", [50, 3]),              # head_dim 48 on the 64-dim layout
    (2, 3, 300, 96, 32, "shuffled", [300, 45]),           # head_dim 96, page = quant block 32
    (2, 2, 200, 112, 64, "interleaved", [200, 64]),       # head_dim 112, page 64
    (2, 2, 50, 24, 16, "contiguous", [50, 9]),            # head_dim 24: the straddling lane loads bytes 8..23
    (2, 3, 300, 72, 32, "shuffled", [300, 45]),           # head_dim 72, two tiles per page
    (2, 2, 60, 20, 16, "interleaved", [60, 13]),          # head_dim 20: the straddling lane loads bytes 4..19
    (2, 3, 300, 44, 32, "shuffled", [300, 45]),           # head_dim 44: 12 dims past 32, two tiles per page
    (2, 2, 200, 196, 16, "contiguous", [200, 77]),        # head_dim 196: 4 dims past 192 on the 256-dim layout
    (2, 2, 60, 18, 16, "interleaved", [60, 13]),          # generic path: head_dim 18
    (3, 4, 200, 128, 8, "shuffled", [200, 17, 9]),        # 8-token pages: two pages per tile
    (2, 2, 100, 64, 8, "interleaved", [100, 8]),          # 8-token pages, 64-dim layout
    (2, 3, 150, 96, 24, "shuffled", [150, 50]),           # 24-token pages
])
def test_paged_attention_matches_oracle(B, H, S, D, page, layout, lengths):
    announce(f"paged B{B} H{H} S{S} D{D} page{page} {layout} lengths={lengths}")
    q, cache = _paged_case(B, H, S, D, page, seed=B * 100 + S, layout=layout, lengths=lengths)
    got, stats = fa.paged_quant_attention_triton(q.to(DEV), cache, return_stats=True)
    sync()
    assert stats["materializes_dense_kv"] == 0.0
    ref = oracle_paged_attention(q, cache)
    if lengths is not None and 0 in lengths:
        keep = [i for i, L in enumerate(lengths) if L != 0]
        assert (got[[i for i in range(B) if i not in keep]] == 0).all()
        got, ref = got[keep], ref[keep]
    assert_attention_close(got, ref, torch.float16, "paged")


@pytest.mark.parametrize("page,qb,D", [(32, 16, 128), (64, 16, 64), (64, 32, 256), (128, 64, 96), (16, 8, 128),
                                       (32, 8, 64), (48, 24, 128)])
def test_paged_pages_holding_several_quant_blocks(page, qb, D):
    """Pages of page // qb quant blocks each (reference triton_paged.py:242-246), shuffled table."""

    announce(f"paged page{page} quant block {qb} D{D}")
    B, H, S = 3, 4, 5 * page + 3
    lengths = np.array([S, page + 1, 2 * page - 5], dtype=np.int64)
    k = np_of(randn((B, H, S, D), 71).float())
    v = np_of(randn((B, H, S, D), 72).float())
    n = -(-S // page)
    rng = np.random.default_rng(page + qb)
    perm = rng.permutation(B * n)
    pk = op.dense_to_pages(k, page)[perm]
    pv = op.dense_to_pages(v, page)[perm]
    table = np.empty(B * n, dtype=np.int64)
    table[perm] = np.arange(B * n)
    cache = op.OracleCache(oq.quantize_int8_per_block(pk, qb), oq.quantize_int8_per_block(pv, qb),
                           table.reshape(B, n), lengths, page, S)
    q = randn((B, H, D), 73)
    got = fa.paged_quant_attention_triton(q.to(DEV), to_cache(cache, DEV))
    assert lib_tiled(D, page, qb)
    assert_attention_close(got, oa.paged_quant_attention(np_of(q), cache), torch.float16, f"page{page} qb{qb}")


def lib_tiled(D, page, qb):
    return bool(_lib.require().fs_decode_tiled_path(D, page, qb))


@pytest.mark.parametrize("q_dtype", [torch.bfloat16, torch.float32])
def test_paged_attention_other_query_dtypes(q_dtype):
    announce(f"paged dtype {q_dtype}")
    q, cache = _paged_case(4, 8, 1000, 128, 16, seed=11, layout="shuffled", lengths=[1000, 999, 500, 16],
                           q_dtype=q_dtype)
    got = fa.paged_quant_attention_triton(q.to(DEV), cache)
    sync()
    assert got.dtype == q_dtype
    assert_attention_close(got, oracle_paged_attention(q, cache), q_dtype, str(q_dtype))


@pytest.mark.parametrize("D,qb,q_dtype", [(128, 16, torch.bfloat16), (120, 16, torch.bfloat16),
                                          (64, 32, torch.bfloat16), (64, 16, torch.float32),
                                          (128, 16, torch.float32), (34, 16, torch.float32)])
def test_query_rows_at_extreme_magnitudes(D, qb, q_dtype):
    """Rows of zeros, of tiny and of huge values, and a row whose one large element sits beside tiny
    ones.  bf16 queries over INT8 blocks enter the fp16 score path scaled by a power of two per row
    (the tiny elements fall to fp16 subnormals or zero); huge rows make the softmax one-hot, which
    holds only if exp2(score - max) sees the same rounded score as the running max (64-dim layout,
    generic kernel at head_dim 34)."""

    announce(f"query magnitudes D{D} qb{qb} {q_dtype}")
    B, H, S = 2, 4, 300
    base = randn((B, H, D), 91, torch.float32)
    rows = [torch.zeros(D), base[0, 1] * 1e-20, base[0, 2] * 1e20, base[0, 3]]
    big = torch.full((D,), 1e-6)
    big[D // 3] = 1e4
    rows += [big, base[1, 1] * 3e-3, base[1, 2] * 40.0, -base[1, 3]]
    q = torch.stack(rows).reshape(B, H, D).to(q_dtype)
    k = randn((B, H, S, D), 92)
    v = randn((B, H, S, D), 93)
    lens = torch.tensor([S, 137], dtype=torch.int64)
    cache = fa.PagedKVCache.from_dense(k.to(DEV), v.to(DEV), block_size=qb, lengths=lens.to(DEV),
                                       block_table_pattern="shuffled", layout_seed=4)
    got = fa.paged_quant_attention_triton(q.to(DEV), cache)
    sync()
    assert lib_tiled(D, qb, qb) == (D % 4 == 0)
    assert_attention_close(got, oracle_paged_attention(q, cache), q_dtype, f"magnitudes D{D} {q_dtype}")


@pytest.mark.parametrize("q_dtype", [torch.float16, torch.bfloat16])
def test_long_rows_split_many_ways(q_dtype):
    """Two heads over ~100k-token rows (6250 tiles): the planner splits each row dozens of ways and
    the splits merge inside the launch; paged (shuffled pages, ragged) and contiguous."""

    announce(f"long rows {q_dtype}")
    B, H, S, D = 1, 2, 100_000, 128
    lens = [99_993]
    q, cache = _paged_case(B, H, S, D, 16, seed=77, layout="shuffled", lengths=lens, q_dtype=q_dtype)
    got, stats = fa.paged_quant_attention_triton(q.to(DEV), cache, return_stats=True)
    sync()
    assert stats["num_splits"] >= 16
    assert_attention_close(got, oracle_paged_attention(q, cache), q_dtype, "long paged")
    k = randn((B, H, S, D), 78)
    v = randn((B, H, S, D), 79)
    kq = oq.quantize_int8_per_block(np_of(k.float()), 16)
    vq = oq.quantize_int8_per_block(np_of(v.float()), 16)
    lt = torch.tensor(lens, dtype=torch.int64)
    got, stats = fa.fused_dequant_attention_triton(q.to(DEV), to_qt(kq, DEV), to_qt(vq, DEV), lengths=lt.to(DEV),
                                                   return_stats=True)
    sync()
    assert stats["num_splits"] >= 16
    assert_attention_close(got, oa.fused_dequant_attention(np_of(q.float()), kq, vq, lt.numpy()), q_dtype, "long fused")


def test_metric_shape_paged_b8_h32_s4096_d128_matches_oracle():
    announce("metric paged B8 H32 S4096 D128")
    q, cache = _paged_case(8, 32, 4096, 128, 16, seed=0)
    got = fa.paged_quant_attention_triton(q.to(DEV), cache)
    sync()
    assert_attention_close(got, oracle_paged_attention(q, cache), torch.float16, "metric")


def test_layouts_and_fused_give_bit_identical_outputs(monkeypatch):
    """Same logical K/V in any physical layout (or contiguous) runs the same arithmetic.

    Every wave sums its tiles in a fixed order, so the results are bit-identical.
    """

    announce("layout invariance B4 H8 S1000 D128")
    k, v, q = randn((4, 8, 1000, 128), 1), randn((4, 8, 1000, 128), 2), randn((4, 8, 128), 3).to(DEV)
    lengths = torch.tensor([1000, 999, 512, 7], device=DEV)
    outs = []
    for layout in ("contiguous", "shuffled", "interleaved"):
        cache = fa.PagedKVCache.from_dense(k.to(DEV), v.to(DEV), 16, lengths=lengths, block_table_pattern=layout)
        outs.append(fa.paged_quant_attention_triton(q, cache))
    kq = fa.quantize_int8_per_block(k.to(DEV), 16)
    vq = fa.quantize_int8_per_block(v.to(DEV), 16)
    outs.append(fa.fused_dequant_attention_triton(q, kq, vq, lengths=lengths))
    sync()
    for o in outs[1:]:
        assert torch.equal(o, outs[0])


def test_multi_split_rows_match_single_split(monkeypatch):
    """Rows split across workgroups (second-launch merge) agree with one split per row."""

    announce("forced splits vs default")
    q, cache = _paged_case(8, 32, 2048, 128, 16, seed=21, layout="shuffled",
                           lengths=[2048, 2000, 1024, 1023, 512, 100, 17, 1])
    single, st1 = fa.paged_quant_attention_triton(q.to(DEV), cache, return_stats=True)
    assert st1["num_splits"] == 1.0
    for n in ("2", "7", "16"):
        monkeypatch.setenv("FLASHSPEC_NUM_SPLITS", n)
        multi, st = fa.paged_quant_attention_triton(q.to(DEV), cache, return_stats=True)
        sync()
        assert st["num_splits"] > 1.0
        assert (multi.float() - single.float()).abs().max().item() <= 2e-3
        assert_attention_close(multi, oracle_paged_attention(q, cache), torch.float16, f"splits={n}")
    for _ in range(3):  # repeated launches are bit-identical
        again = fa.paged_quant_attention_triton(q.to(DEV), cache)
        sync()
        assert torch.equal(again, multi)


@pytest.mark.parametrize("warps", ["1", "2", "4", "8"])
def test_waves_per_block_knob(monkeypatch, warps):
    announce(f"num_warps={warps}")
    q, cache = _paged_case(2, 8, 900, 128, 16, seed=31, lengths=[900, 450])
    base = fa.paged_quant_attention_triton(q.to(DEV), cache)
    monkeypatch.setenv("FLASHSPEC_NUM_WARPS", warps)
    other, stats = fa.paged_quant_attention_triton(q.to(DEV), cache, return_stats=True)
    sync()
    assert stats["num_warps"] == float(warps)
    assert (base.float() - other.float()).abs().max().item() <= 2e-3
    assert_attention_close(other, oracle_paged_attention(q, cache), torch.float16, f"warps={warps}")


def test_repeated_calls_are_bit_identical():
    """Fixed per-wave tile order: the metric-shape decode is bit-reproducible."""

    announce("bit-reproducibility B8 H32 S4096")
    q, cache = _paged_case(8, 32, 4096, 128, 16, seed=71, layout="shuffled")
    outs = [fa.paged_quant_attention_triton(q.to(DEV), cache) for _ in range(4)]
    sync()
    for o in outs[1:]:
        assert torch.equal(o, outs[0])


def test_unallocated_pages_and_lengths_past_the_table_are_masked():
    """A -1 table entry inside a row's length: the HIP kernel masks that page's tokens (the
    reference Triton kernel's semantics, triton_paged.py:219-232), whereas the reference PyTorch
    path reads physical page 0 there (paged.py:441, ``block_table.clamp_min(0)``).  Both are run
    on the same cache: rows without such an entry match the oracle; the affected row equals the
    oracle's attention over the backed tokens only, and differs from the page-0 reading.  A length
    past max_seq_len is clamped to it, as in both reference paths."""

    announce("table -1 entries / clamped lengths")
    q, cache = _paged_case(2, 4, 64, 128, 16, seed=41)
    table = cache.block_table.clone()
    table[1, 1] = -1  # row 1: tokens [16, 32) have no backing page
    lengths = torch.tensor([999, 64], device=DEV)  # row 0 clamps to max_seq_len
    masked = fa.PagedKVCache(cache.k_quant, cache.v_quant, table, lengths, 16, 64)
    got = fa.paged_quant_attention_triton(q.to(DEV), masked)
    sync()
    # the reference PyTorch path on the identical cache (page 0 read for the -1 entry)
    same = oracle_paged_attention(q, masked)
    assert_attention_close(got[:1], same[:1], torch.float16, "row without -1 entries")
    # row 1 as documented: attention over tokens [0, 16) and [32, 64) only
    dense = op.to_dense(from_cache(masked))
    keep = np.r_[0:16, 32:64]
    k1 = dense[0][1:2][:, :, keep]
    v1 = dense[1][1:2][:, :, keep]
    want = oa.reference_attention(np_of(q)[1:2].astype(np.float32), k1, v1)
    assert_attention_close(got[1:], want, torch.float16, "row with a -1 entry")
    diverge = np.abs(got[1:].float().cpu().numpy() - cast_like_q(same[1:], torch.float16)).max()
    assert diverge > 1e-2, "the page-0 reading of the reference PyTorch path should differ on this row"


def test_graph_replay_matches_eager():
    announce("graph capture/replay paged attention")
    q, cache = _paged_case(8, 32, 1024, 128, 16, seed=51, layout="shuffled")
    qd = q.to(DEV)
    eager = fa.paged_quant_attention_triton(qd, cache)
    sync()
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream(DEV)
    stream.wait_stream(torch.cuda.current_stream(DEV))
    with torch.cuda.stream(stream):
        fa.paged_quant_attention_triton(qd, cache)  # warm up on the capture stream
        stream.synchronize()
        with torch.cuda.graph(graph, stream=stream):
            out = fa.paged_quant_attention_triton(qd, cache)
    torch.cuda.current_stream(DEV).wait_stream(stream)
    for i in range(4):
        graph.replay()
        sync()
        scratch = torch.randn(1024, device=DEV).sum()  # eager work between replays
        sync()
        assert torch.equal(out, eager), f"replay {i}"
        del scratch


def test_gpu_validation_errors_before_launch():
    announce("validation errors")
    q, cache = _paged_case(2, 4, 64, 128, 16, seed=61)
    with pytest.raises(ValueError):
        fa.paged_quant_attention_triton(q[:, :2].to(DEV), cache)
    with pytest.raises(ValueError):
        fa.paged_quant_attention_triton(q.to(DEV).to(torch.float64), cache)
    kq = fa.quantize_int8_per_block(randn((2, 4, 64, 128), 1).to(DEV))
    with pytest.raises(ValueError):
        fa.fused_dequant_attention_triton(q.to(DEV), kq, kq, lengths=torch.tensor([1, 2, 3], device=DEV))
    with pytest.raises(RuntimeError):
        fa.fused_dequant_attention_triton(q.to(DEV), kq, kq, lengths=torch.tensor([1, 2]))


def test_repeat_launch_memo_still_validates_and_stays_correct():
    """Repeated launches over one cache skip re-validation only for an identical signature:
    a changed query, a different V store or lengths of another shape are checked again."""

    announce("repeat-launch layout memo: paged + fused, mismatches after a good call")
    k = randn((2, 4, 100, 64), 31)
    v = randn((2, 4, 100, 64), 32)
    q = randn((2, 4, 64), 33)
    cache = fa.PagedKVCache.from_dense(k.to(DEV), v.to(DEV), block_size=16, block_table_pattern="shuffled",
                                       layout_seed=3)
    ref = oracle_paged_attention(q, cache)
    for _ in range(3):
        out = fa.paged_quant_attention_triton(q.to(DEV), cache)
        sync()
        assert_attention_close(out, ref, q.dtype, "paged repeat")
    with pytest.raises(ValueError):
        fa.paged_quant_attention_triton(randn((2, 3, 64), 34).to(DEV), cache)
    with pytest.raises(ValueError):
        fa.paged_quant_attention_triton(randn((2, 4, 64), 34).to(DEV).float().to(torch.float64), cache)
    out = fa.paged_quant_attention_triton(q.to(DEV), cache)
    sync()
    assert_attention_close(out, ref, q.dtype, "paged after rejected calls")
    # a second cache of another length through the same process-wide plan memo
    cache2 = fa.PagedKVCache.from_dense(k[:, :, :37].to(DEV), v[:, :, :37].to(DEV), block_size=16)
    out2 = fa.paged_quant_attention_triton(q.to(DEV), cache2)
    sync()
    assert_attention_close(out2, oracle_paged_attention(q, cache2), q.dtype, "second cache")

    kq = fa.quantize_int8_per_block(k.to(DEV), 16)
    vq = fa.quantize_int8_per_block(v.to(DEV), 16)
    fref = oracle_fused_attention(q, kq, vq)
    for _ in range(2):
        out = fa.fused_dequant_attention_triton(q.to(DEV), kq, vq)
        sync()
        assert_attention_close(out, fref, q.dtype, "fused repeat")
    v_short = fa.quantize_int8_per_block(v[:, :, :50].to(DEV), 16)
    with pytest.raises(ValueError):
        fa.fused_dequant_attention_triton(q.to(DEV), kq, v_short)
    with pytest.raises(ValueError):
        fa.fused_dequant_attention_triton(q.to(DEV), kq, vq, torch.tensor([100, 100, 100], device=DEV))
    lengths = torch.tensor([100, 41], device=DEV)
    out = fa.fused_dequant_attention_triton(q.to(DEV), kq, vq, lengths)
    sync()
    assert_attention_close(out, oracle_fused_attention(q, kq, vq, lengths.cpu()), q.dtype, "fused with lengths")
