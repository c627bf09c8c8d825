"""Host-side API tests on CPU tensors.

These restate the reference's own unit tests (reference tests/test_flashspec.py)
against flashspec_amd: CPU tensors take the portable path, which must keep the
reference's semantics, and the accelerated entry points must fall back exactly
like the reference's "fake backend" (triton_utils.py:65-73).  Also covers the
knob resolvers the reference pins, the split planner and error classes.
"""

from __future__ import annotations

import os

import numpy as np
import pytest
import torch

import flashspec_amd as fa
import flashspec_amd.triton_fused as triton_fused
import flashspec_amd.triton_paged as triton_paged
from flashspec_amd import (
    PagedKVAllocator,
    PagedKVCache,
    dequantize_int8_per_block,
    fused_dequant_attention,
    fused_dequant_attention_triton,
    paged_quant_attention,
    paged_quant_attention_triton,
    quantize_int8_per_block,
    reference_attention,
)
from flashspec_amd import triton_utils
from oracle import attention as oa
from oracle import quant as oq
from tests._helpers import assert_quant_equal, from_qt, golden_cache, load_npz, np_of, to_cache


@pytest.fixture(autouse=True)
def _seed():
    torch.manual_seed(7)


@pytest.fixture
def clean_env(monkeypatch):
    for key in ("FLASHSPEC_NUM_SPLITS", "FLASHSPEC_BLOCK_N", "FLASHSPEC_NUM_WARPS"):
        monkeypatch.delenv(key, raising=False)
    return monkeypatch


def test_quant_round_trip_has_bounded_error():
    x = torch.randn(2, 3, 19, 16)
    q = quantize_int8_per_block(x, block_size=8)
    y = dequantize_int8_per_block(q)
    assert tuple(y.shape) == tuple(x.shape)
    assert float((x - y).abs().max()) < 0.03


def test_portable_quantizer_is_bit_exact_with_reference_vectors():
    d = load_npz("quant_golden.npz")
    for name in d["names"]:
        x = torch.from_numpy(d[f"{name}_x"])
        q = quantize_int8_per_block(x, block_size=int(d[f"{name}_block"]))
        assert_quant_equal(from_qt(q), oq.OracleQuant(d[f"{name}_values"], d[f"{name}_scale"], d[f"{name}_zero"],
                                                       0, ()), name)


def test_fused_dequant_attention_matches_dequant_reference():
    q = torch.randn(2, 3, 16)
    k = torch.randn(2, 3, 25, 16)
    v = torch.randn(2, 3, 25, 16)
    kq, vq = quantize_int8_per_block(k, block_size=8), quantize_int8_per_block(v, block_size=8)
    expected = reference_attention(q, dequantize_int8_per_block(kq), dequantize_int8_per_block(vq))
    torch.testing.assert_close(fused_dequant_attention(q, kq, vq), expected, rtol=1e-5, atol=1e-5)
    # and the portable path agrees with the numpy oracle
    np.testing.assert_allclose(np_of(expected), oa.fused_dequant_attention(np_of(q), from_qt(kq), from_qt(vq)),
                               rtol=1e-5, atol=1e-5)


def test_triton_fused_wrapper_falls_back_on_cpu():
    q = torch.randn(2, 3, 16)
    k = torch.randn(2, 3, 25, 16)
    v = torch.randn(2, 3, 25, 16)
    kq, vq = quantize_int8_per_block(k, block_size=8), quantize_int8_per_block(v, block_size=8)
    expected = fused_dequant_attention(q, kq, vq)
    actual, stats = fused_dequant_attention_triton(q, kq, vq, return_stats=True)
    torch.testing.assert_close(actual, expected, rtol=1e-5, atol=1e-5)
    assert stats["materializes_dense_kv"] == 1.0


def test_default_knobs_match_reference(clean_env):
    assert triton_fused._resolve_block_n() == 128
    assert triton_fused._resolve_num_warps() == 4
    assert triton_fused._compute_num_splits(seq_len=2048, block_n=128) == 4
    assert triton_fused._compute_num_splits(seq_len=4096, block_n=128) == 4
    assert triton_fused._compute_num_splits(seq_len=512, block_n=128) == 1
    assert triton_paged._resolve_block_n() == 128
    assert triton_paged._resolve_num_warps() == 4
    clean_env.setenv("FLASHSPEC_BLOCK_N", "64")
    clean_env.setenv("FLASHSPEC_NUM_WARPS", "8")
    clean_env.setenv("FLASHSPEC_NUM_SPLITS", "1")
    assert triton_fused._resolve_block_n() == 64
    assert triton_fused._resolve_num_warps() == 8
    assert triton_fused._compute_num_splits(seq_len=2048, block_n=64) == 1
    assert triton_paged._resolve_block_n() == 64
    assert triton_paged._resolve_num_warps() == 8
    clean_env.setenv("FLASHSPEC_BLOCK_N", "48")  # invalid values fall back to the defaults
    clean_env.setenv("FLASHSPEC_NUM_WARPS", "3")
    assert triton_fused._resolve_block_n() == 128 and triton_fused._resolve_num_warps() == 4


def test_contiguous_rows_at_head_dim_64_plan_eight_waves(clean_env):
    """The default plan for contiguous rows at head_dim 64 takes 8-wave workgroups; paged rows, the
    tail head_dims that share the 64-dim layout and a forced wave count keep their own."""

    from flashspec_amd import _lib

    _lib.require()  # the tiled-path rule is a host function of the library
    clean_env.setitem(triton_utils._CU_CACHE, 0, 256)
    triton_utils._launch_plan_cached.cache_clear()
    plan = triton_utils.launch_plan
    dev = torch.device("cuda", 0)
    assert plan(4096, 256, 64, 16, 16, dev, contiguous=True) == (True, 8, 256, 1, 128)
    assert plan(4096, 256, 64, 16, 16, dev) == (True, 16, 256, 1, 128)
    assert plan(4096, 256, 48, 16, 16, dev, contiguous=True)[1] == 16
    assert plan(4096, 256, 128, 16, 16, dev, contiguous=True)[1] == 16
    tiled, waves, split_tiles, max_splits, _ = plan(8192, 64, 64, 16, 16, dev, contiguous=True)
    assert (waves, max_splits) == (8, 4) and split_tiles * max_splits >= 512
    clean_env.setenv("FLASHSPEC_NUM_WARPS", "16")
    assert plan(4096, 256, 64, 16, 16, dev, contiguous=True)[1] == 16
    triton_utils._launch_plan_cached.cache_clear()


def test_split_plan_covers_every_tile(clean_env):
    for tiled in (True, False):
        for seq_len in (1, 15, 16, 17, 129, 1500, 2048, 4096, 16384, 65536):
            for rows in (1, 8, 128, 256, 2048):
                for fixed in (None, 1, 16):
                    split_tiles, max_splits, waves = triton_utils.plan_splits(seq_len, rows, 128, 256, tiled=tiled,
                                                                              waves=fixed)
                    tiles = -(-seq_len // 16)
                    assert split_tiles >= 1 and max_splits >= 1 and waves in (1, 2, 4, 8, 16)
                    assert split_tiles * max_splits >= tiles > split_tiles * (max_splits - 1)
                    if tiled:
                        assert split_tiles <= 64 * waves
                        if fixed:
                            assert waves == fixed
    # per-channel stores: splits hold whole quant blocks of `grp` tiles, a wave at most 64 tiles
    for grp in (2, 3, 4, 8, 64):
        for seq_len in (1, 17, 300, 1000, 4096, 65536):
            for rows in (1, 8, 256):
                for fixed in (None, 1, 8):
                    split_tiles, max_splits, waves = triton_utils.plan_splits(
                        seq_len, rows, 128, 256, waves=fixed, max_waves=8, tile_group=grp)
                    tiles = -(-seq_len // 16)
                    assert split_tiles % grp == 0 and waves in (1, 2, 4, 8)
                    assert grp * -(-(split_tiles // grp) // waves) <= 64
                    assert split_tiles * max_splits >= tiles > split_tiles * (max_splits - 1)
    assert triton_utils.plan_splits(4096, 256, 128, 256, max_waves=8, tile_group=4) == (256, 1, 8)
    plan = triton_utils.plan_splits
    # metric shape: 256 rows on 256 CUs -> one 16-wave workgroup per row, no second launch
    assert plan(4096, 256, 128, 256) == (256, 1, 16)
    # light tiles (fp16 query over INT8 blocks, 128-dim layout): 4-wave workgroups when one
    # workgroup lands on 3/4 to all of the CUs and every wave keeps 32..64 tiles
    assert plan(4096, 256, 128, 256, light=True) == (256, 1, 4)
    assert plan(2048, 256, 128, 256, light=True) == (128, 1, 4)
    assert plan(8192, 128, 128, 256, light=True) == (256, 2, 4)
    assert plan(4096, 128, 128, 256, light=True) == (128, 2, 4)
    assert plan(16384, 32, 128, 256, light=True) == (128, 8, 4)
    assert plan(4096, 512, 128, 256, light=True) == (256, 1, 16)   # two workgroups per CU
    assert plan(8192, 256, 128, 256, light=True) == (512, 1, 16)   # 4 waves would need a second split
    assert plan(1024, 256, 128, 256, light=True) == (64, 1, 4)     # short rows: 16 tiles per wave
    assert plan(4096, 64, 128, 256, light=True) == (64, 4, 4)      # 4 splits of 64 tiles, merged in-kernel
    assert plan(512, 256, 128, 256, light=True) == (32, 1, 8)      # under 64 tiles: the general rule
    assert plan(4096, 96, 128, 256, light=True) == (86, 3, 16)
    assert plan(4096, 160, 128, 256, light=True) == (128, 2, 16)   # 320 workgroups: more than one per CU
    clean_env.setenv("FLASHSPEC_NUM_SPLITS", "1")  # 128 of 256 CUs busy: not full enough for 4 waves
    assert plan(2048, 128, 128, 256, light=True) == (128, 1, 16)
    # forced split counts of 2+: at most 8 waves per workgroup (in-kernel merge) and, with more
    # workgroups than CUs, about 8 resident waves per CU; enough for a split's tiles
    clean_env.setenv("FLASHSPEC_NUM_SPLITS", "4")
    assert plan(4096, 256, 128, 256, light=True) == (64, 4, 2)     # the reference's C2 setting
    assert plan(4096, 256, 128, 256) == (64, 4, 2)
    assert plan(2048, 128, 128, 256, light=True) == (32, 4, 4)
    assert plan(16384, 32, 128, 256, light=True) == (256, 4, 8)
    clean_env.setenv("FLASHSPEC_NUM_SPLITS", "2")
    assert plan(4096, 256, 128, 256, light=True) == (128, 2, 4)
    assert plan(65536, 256, 128, 256, light=True) == (1024, 4, 16)  # 2048-tile splits need 32 waves
    clean_env.setenv("FLASHSPEC_NUM_SPLITS", "8")
    assert plan(4096, 256, 128, 256, light=True) == (32, 8, 1)
    clean_env.delenv("FLASHSPEC_NUM_SPLITS")
    clean_env.setenv("FLASHSPEC_NUM_WARPS", "16")
    assert plan(4096, 256, 128, 256, waves=triton_utils.forced_tiled_waves(), light=True) == (256, 1, 16)
    clean_env.delenv("FLASHSPEC_NUM_WARPS")
    # half the CUs hold a row: split in two only when each half keeps 128 tiles (64 for light
    # tiles, whose 4-wave splits merge in-kernel), else run unsplit with 8 waves (C1: B4 H32 S2048)
    assert plan(2048, 128, 128, 256) == (128, 1, 8)
    assert plan(4096, 128, 128, 256) == (128, 2, 16)
    assert plan(2048, 128, 128, 256, light=True) == (64, 2, 4)
    assert plan(1024, 128, 128, 256, light=True) == (64, 1, 8)     # halves of 32 tiles: unsplit
    # few rows: split rows to fill the GPU; workgroup size follows the split length
    assert plan(2048, 64, 128, 256) == (32, 4, 8)
    assert plan(1500, 8, 128, 256) == (8, 12, 2)   # the reference's split-K test shape splits
    assert plan(4096, 8, 128, 256) == (8, 32, 2)
    clean_env.setenv("FLASHSPEC_NUM_SPLITS", "1")
    assert plan(4096, 256, 128, 256) == (256, 1, 16)
    clean_env.setenv("FLASHSPEC_NUM_SPLITS", "1000")  # clamped to ceil(S/block_n); 8192 workgroups of 1 wave
    assert plan(4096, 256, 128, 256) == (8, 32, 1)
    clean_env.setenv("FLASHSPEC_NUM_WARPS", "8")
    assert triton_utils.forced_tiled_waves() == 8
    clean_env.setenv("FLASHSPEC_NUM_WARPS", "16")
    assert triton_utils.forced_tiled_waves() == 16 and triton_utils.resolve_num_warps() == 4


def test_paged_cache_reconstructs_dense_quantized_kv():
    k = torch.randn(2, 4, 23, 8)
    v = torch.randn(2, 4, 23, 8)
    cache = PagedKVCache.from_dense(k, v, block_size=6)
    kd, vd = cache.to_dense()
    assert tuple(kd.shape) == tuple(k.shape) and tuple(vd.shape) == tuple(v.shape)
    assert float((k - kd).abs().max()) < 0.03 and float((v - vd).abs().max()) < 0.03


def test_paged_cache_profile_layouts_preserve_logical_kv():
    k = torch.randn(3, 2, 17, 8)
    v = torch.randn(3, 2, 17, 8)
    lengths = torch.tensor([17, 11, 5], dtype=torch.int64)
    for layout in ("shuffled", "interleaved"):
        cache = PagedKVCache.from_dense(k, v, block_size=4, lengths=lengths, block_table_pattern=layout,
                                        layout_seed=13)
        kd, vd = cache.to_dense()
        assert tuple(cache.lengths.tolist()) == tuple(lengths.tolist())
        assert float((k - kd).abs().max()) < 0.03 and float((v - vd).abs().max()) < 0.03


def test_portable_layouts_match_reference_golden_tables():
    d = load_npz("layout_golden.npz")
    k, v, lengths = (torch.from_numpy(d[x]) for x in ("k", "v", "lengths"))
    for key, layout, seed in (("contiguous0", "contiguous", 0), ("shuffled13", "shuffled", 13),
                              ("shuffled0", "shuffled", 0), ("interleaved0", "interleaved", 0)):
        cache = PagedKVCache.from_dense(k, v, block_size=4, lengths=lengths, block_table_pattern=layout,
                                        layout_seed=seed)
        ref = golden_cache(d, key)
        assert np.array_equal(np_of(cache.block_table), ref.block_table), key
        assert_quant_equal(from_qt(cache.k_quant), ref.k_quant, key)


def test_paged_attention_matches_dense_quant_attention():
    q = torch.randn(2, 2, 8)
    k = torch.randn(2, 2, 17, 8)
    v = torch.randn(2, 2, 17, 8)
    cache = PagedKVCache.from_dense(k, v, block_size=4)
    kd, vd = cache.to_dense()
    expected = reference_attention(q, kd, vd, lengths=cache.lengths)
    torch.testing.assert_close(paged_quant_attention(q, cache), expected, rtol=1e-5, atol=1e-5)


def test_triton_paged_wrapper_falls_back_on_cpu():
    q = torch.randn(2, 2, 8)
    cache = PagedKVCache.from_dense(torch.randn(2, 2, 17, 8), torch.randn(2, 2, 17, 8), block_size=4)
    expected = paged_quant_attention(q, cache)
    actual, stats = paged_quant_attention_triton(q, cache, return_stats=True)
    torch.testing.assert_close(actual, expected, rtol=1e-5, atol=1e-5)
    assert stats["materializes_dense_kv"] == 1.0
    assert stats["physical_blocks"] == 10.0


def test_paged_cache_append_extends_cache_without_dense_rebuild():
    k, v = torch.randn(2, 2, 5, 8), torch.randn(2, 2, 5, 8)
    k_new, v_new = torch.randn(2, 2, 3, 8), torch.randn(2, 2, 3, 8)
    appended = PagedKVCache.from_dense(k, v, block_size=4).append(k_new, v_new)
    kd, vd = appended.to_dense()
    assert tuple(appended.lengths.tolist()) == (8, 8)
    assert float((torch.cat([k, k_new], 2) - kd).abs().max()) < 0.06
    assert float((torch.cat([v, v_new], 2) - vd).abs().max()) < 0.06


def test_portable_append_is_bit_exact_with_reference_vectors():
    d = load_npz("append_golden.npz")
    for name in d["names"]:
        cin = to_cache(golden_cache(d, f"{name}_in"), "cpu")
        ref = golden_cache(d, f"{name}_out")
        out = cin.append(torch.from_numpy(d[f"{name}_kn"]), torch.from_numpy(d[f"{name}_vn"]))
        assert np.array_equal(np_of(out.block_table), ref.block_table), name
        assert_quant_equal(from_qt(out.k_quant), ref.k_quant, name)
        assert_quant_equal(from_qt(out.v_quant), ref.v_quant, name)


def test_paged_attention_after_append_matches_reconstructed_cache():
    q = torch.randn(2, 2, 8)
    cache = PagedKVCache.from_dense(torch.randn(2, 2, 7, 8), torch.randn(2, 2, 7, 8), block_size=4)
    cache = cache.append(torch.randn(2, 2, 2, 8), torch.randn(2, 2, 2, 8))
    kd, vd = cache.to_dense()
    torch.testing.assert_close(paged_quant_attention(q, cache), reference_attention(q, kd, vd, cache.lengths),
                               rtol=1e-5, atol=1e-5)


def test_paged_allocator_append_release_and_reuse():
    allocator = PagedKVAllocator(capacity_blocks=6, heads=2, head_dim=8, block_size=4)
    k0, v0 = torch.randn(1, 2, 5, 8), torch.randn(1, 2, 5, 8)
    allocator.add_request(10, k0, v0)
    allocator.add_request(20, torch.randn(1, 2, 3, 8), torch.randn(1, 2, 3, 8))
    released = int(allocator.to_cache([10, 20]).block_table[1, 0])
    assert allocator.stats()["allocated_blocks"] == 3.0
    k_new, v_new = torch.randn(1, 2, 4, 8), torch.randn(1, 2, 4, 8)
    allocator.append_request(10, k_new, v_new)
    appended = allocator.to_cache([10])
    kd, vd = appended.to_dense()
    assert tuple(appended.lengths.tolist()) == (9,)
    assert allocator.stats()["allocated_blocks"] == 4.0
    assert float((torch.cat([k0, k_new], 2) - kd).abs().max()) < 0.08
    allocator.release_request(20)
    allocator.add_request(30, torch.randn(1, 2, 1, 8), torch.randn(1, 2, 1, 8))
    assert int(allocator.to_cache([30]).block_table[0, 0]) == released
    assert "fragmentation" in allocator.stats()


def test_portable_allocator_is_bit_exact_with_reference_vectors():
    d = load_npz("allocator_golden.npz")
    H, D, bs, cap = (int(x) for x in d["config"])
    alloc = PagedKVAllocator(capacity_blocks=cap, heads=H, head_dim=D, block_size=bs)
    for step, (code, rid, _n) in enumerate(d["script"]):
        if code == 0:
            alloc.add_request(int(rid), torch.from_numpy(d[f"s{step}_k"]), torch.from_numpy(d[f"s{step}_v"]))
        elif code == 1:
            alloc.append_request(int(rid), torch.from_numpy(d[f"s{step}_k"]), torch.from_numpy(d[f"s{step}_v"]))
        else:
            alloc.release_request(int(rid))
        assert np.array_equal(np_of(alloc.k_quant.values), d[f"s{step}_kvalues"]), step
        assert np.array_equal(np_of(alloc.v_quant.scale).view(np.uint32), d[f"s{step}_vscale"].view(np.uint32))


def test_symmetric_per_token_format_portable_paths():
    """quantize_int8_symmetric_per_token is bit-exact with the oracle, and the block-1 affine
    layout it returns flows through fused, paged (all layouts) and dequantize unchanged."""

    g = torch.Generator().manual_seed(21)
    k = torch.randn((2, 3, 37, 32), generator=g) * 2
    v = torch.randn((2, 3, 37, 32), generator=g)
    q = torch.randn((2, 3, 32), generator=g)
    kq = fa.quantize_int8_symmetric_per_token(k)
    ref = oq.quantize_int8_symmetric_per_token(k.numpy())
    assert np.array_equal(kq.values.numpy(), ref.values)
    assert np.array_equal(kq.scale.numpy().view(np.uint32), ref.scale.view(np.uint32))
    assert np.array_equal(kq.zero_point.numpy(), ref.zero_point)
    assert np.array_equal(fa.dequantize_int8_per_block(kq).numpy(), oq.dequantize_int8_per_block(ref))
    vq = fa.quantize_int8_symmetric_per_token(v)
    fused = fa.fused_dequant_attention_triton(q, kq, vq)
    for pattern in ("contiguous", "shuffled", "interleaved"):
        cache = fa.PagedKVCache.from_dense(k, v, 16, block_table_pattern=pattern, kv_format="symmetric_token")
        assert cache.k_quant.block_size == 1
        torch.testing.assert_close(fa.paged_quant_attention_triton(q, cache), fused, rtol=1e-5, atol=1e-5)
    with pytest.raises(ValueError):
        fa.PagedKVCache.from_dense(k, v, 16, kv_format="fp8")


def test_validation_errors_match_reference_classes():
    with pytest.raises(ValueError):
        quantize_int8_per_block(torch.randn(4), 16)
    with pytest.raises(ValueError):
        quantize_int8_per_block(torch.randn(2, 4), 0)
    with pytest.raises(ValueError):
        PagedKVCache.from_dense(torch.randn(1, 1, 4, 8), torch.randn(1, 1, 5, 8))
    with pytest.raises(ValueError):
        PagedKVCache.from_dense(torch.randn(1, 1, 4, 8), torch.randn(1, 1, 4, 8), block_table_pattern="zigzag")
    with pytest.raises(ValueError):
        PagedKVCache.from_dense(torch.randn(2, 1, 4, 8), torch.randn(2, 1, 4, 8), lengths=torch.tensor([5, 1]))
    alloc = PagedKVAllocator(capacity_blocks=1, heads=1, head_dim=8, block_size=4)
    with pytest.raises(RuntimeError):
        alloc.add_request(1, torch.randn(1, 1, 5, 8), torch.randn(1, 1, 5, 8))
    with pytest.raises(KeyError):
        alloc.append_request(7, torch.randn(1, 1, 1, 8), torch.randn(1, 1, 1, 8))
    with pytest.raises(ValueError):
        reference_attention(torch.randn(1, 1, 1, 8), torch.randn(1, 1, 4, 8), torch.randn(1, 1, 4, 8))


def test_validate_decode_query_rejects_cpu_and_wide_heads():
    with pytest.raises(RuntimeError):
        triton_utils.validate_decode_query(torch.randn(1, 1, 8), kernel_name="paged")
    with pytest.raises(ValueError):
        triton_utils.validate_decode_query(torch.randn(1, 8), kernel_name="paged")


def test_compat_aliases_flashspec_names():
    import sys

    import flashspec_amd
    import flashspec_amd.compat  # noqa: F401

    import flashspec  # noqa: F401  (resolves to flashspec_amd)

    assert sys.modules["flashspec"] is flashspec_amd
    assert sys.modules["flashspec.triton_paged"] is triton_paged
    from flashspec.triton_utils import HAS_TRITON

    assert HAS_TRITON == triton_utils.HAS_HIP
