"""Host logic of the serving pieces on CPU: DecodeBatch page reservation, append and
close against the oracle allocator (reference src/flashspec/paged.py:108-151, 221-255),
and the decode simulation's lifecycle (serving.py:33-190).

Every comparison of quantized pages is bit-exact.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import flashspec_amd as fa
from flashspec_amd.serving import DecodeBatch, ServingConfig, build_request_pool, run_decode_simulation
from oracle import paged as op

from tests._helpers import assert_attention_close, from_qt, oracle_paged_attention


def _pair(seed, shape):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g), torch.randn(shape, generator=g)


def _mirror(heads=2, dim=8, page=4, capacity=48, shuffle_seed=5):
    alloc = fa.PagedKVAllocator(capacity_blocks=capacity, heads=heads, head_dim=dim, block_size=page)
    oracle = op.OracleAllocator(capacity, heads, dim, page)
    if shuffle_seed is not None:
        alloc.shuffle_free_blocks(shuffle_seed)
        oracle.free = list(alloc._free_blocks)
    return alloc, oracle


def _add(alloc, oracle, rid, length, seed, heads=2, dim=8):
    k, v = _pair(seed, (1, heads, length, dim))
    alloc.add_request(rid, k, v)
    oracle.add_request(rid, k.numpy(), v.numpy())


def _assert_stores_equal(alloc, oracle):
    for ours, ref, name in ((alloc.k_quant, oracle.k_quant, "K"), (alloc.v_quant, oracle.v_quant, "V")):
        got = from_qt(ours)
        np.testing.assert_array_equal(got.values, ref.values, err_msg=f"{name} values")
        np.testing.assert_array_equal(got.scale, ref.scale, err_msg=f"{name} scale")
        np.testing.assert_array_equal(got.zero_point, ref.zero_point, err_msg=f"{name} zero point")


@pytest.mark.parametrize("shuffle_seed", [None, 5])
def test_decode_batch_matches_oracle_allocator(shuffle_seed):
    alloc, oracle = _mirror(shuffle_seed=shuffle_seed)
    for rid, (length, seed) in enumerate([(5, 1), (8, 2), (3, 3), (12, 4)]):
        _add(alloc, oracle, rid, length, seed)
    # a released request leaves stale rows behind in pages that the batch reuses
    alloc.release_request(1)
    oracle.release_request(1)
    _add(alloc, oracle, 7, 2, 9)
    rids = [0, 2, 3, 7]
    batch = DecodeBatch(alloc, rids, max_new_tokens=9, reserve_steps=4)
    for step in range(9):
        k_new, v_new = _pair(100 + step, (len(rids), 2, 1, 8))
        batch.append(k_new, v_new)
        oracle.append_batch(rids, k_new.numpy(), v_new.numpy())
        _assert_stores_equal(alloc, oracle)
        ref_cache = oracle.to_cache(rids)
        cache = batch.cache()
        np.testing.assert_array_equal(cache.lengths.numpy(), ref_cache.lengths)
        for i in range(len(rids)):
            used = -(-int(ref_cache.lengths[i]) // 4)
            np.testing.assert_array_equal(cache.block_table[i, :used].numpy(), ref_cache.block_table[i, :used])
        q = torch.randn((len(rids), 2, 8), generator=torch.Generator().manual_seed(step))
        assert_attention_close(batch.attend(q), oracle_paged_attention(q, cache), q.dtype, f"step {step}")
    with pytest.raises(RuntimeError, match="opened for 9"):
        batch.append(*_pair(0, (len(rids), 2, 1, 8)))
    batch.close()
    assert alloc._free_blocks == oracle.free
    for rid in rids:
        assert alloc._requests[rid].logical_blocks == oracle.requests[rid]["blocks"]
        assert alloc._requests[rid].length == oracle.requests[rid]["length"]


def test_decode_batch_close_returns_unused_reservations():
    alloc, oracle = _mirror(shuffle_seed=3)
    _add(alloc, oracle, 0, 4, 1)
    _add(alloc, oracle, 1, 6, 2)
    free_before = list(alloc._free_blocks)
    batch = DecodeBatch(alloc, [0, 1], max_new_tokens=20, reserve_steps=8)
    assert len(alloc._free_blocks) < len(free_before)
    k_new, v_new = _pair(7, (2, 2, 1, 8))
    batch.append(k_new, v_new)
    oracle.append_batch([0, 1], k_new.numpy(), v_new.numpy())
    batch.close()
    # request 0 crossed into a new page (length 4 -> 5), request 1 did not (6 -> 7)
    assert alloc._free_blocks == oracle.free
    assert alloc._requests[0].logical_blocks == oracle.requests[0]["blocks"]
    with pytest.raises(RuntimeError, match="closed"):
        batch.append(k_new, v_new)


def test_decode_batch_rejects_bad_inputs():
    alloc, _ = _mirror()
    k, v = _pair(0, (1, 2, 5, 8))
    alloc.add_request(0, k, v)
    with pytest.raises(ValueError):
        DecodeBatch(alloc, [], max_new_tokens=1)
    with pytest.raises(ValueError):
        DecodeBatch(alloc, [0, 0], max_new_tokens=1)
    with pytest.raises(KeyError):
        DecodeBatch(alloc, [3], max_new_tokens=1)
    batch = DecodeBatch(alloc, [0], max_new_tokens=2)
    with pytest.raises(ValueError, match="shape"):
        batch.append(*_pair(0, (1, 2, 2, 8)))


def test_build_request_pool_scatters_pages():
    alloc, rids = build_request_pool([37, 5, 64], heads=2, head_dim=8, block_size=4, headroom_tokens=4, seed=2,
                                     device="cpu", dtype=torch.float32)
    assert rids == [0, 1, 2]
    pages = [p for r in rids for p in alloc._requests[r].logical_blocks]
    assert len(set(pages)) == len(pages) == 10 + 2 + 16
    assert pages != sorted(pages)
    assert alloc.capacity_blocks == 11 + 3 + 17


def test_simulation_counts_arrivals_and_finishes():
    res = run_decode_simulation(ServingConfig(requests=3, prompt_lens=(6, 9), decode_steps=5, request_life_steps=2,
                                              heads=2, head_dim=8, block_size=4, device="cpu", dtype="float32"))
    # every request lives 2 steps: finishes after steps 2 and 4 (3 each), arrivals replace them
    assert res["finishes"] == 6
    assert res["arrivals"] == 9
    assert res["generated_tokens"] == 15
    assert res["live_requests"] == 3.0
    assert res["attention_backend"] == "portable"


def test_decode_batch_failed_reservation_leaves_allocator_unchanged():
    """Opening a batch whose first reservation runs out of pages raises and hands every page it
    took back: free list (order included), request pages and stats are as before."""

    alloc = fa.PagedKVAllocator(capacity_blocks=5, heads=2, head_dim=8, block_size=4)
    for rid in range(3):
        k, v = _pair(rid, (1, 2, 4, 8))  # one full page each
        alloc.add_request(rid, k, v)
    free_before = list(alloc._free_blocks)
    pages_before = {rid: list(alloc._get_request(rid).logical_blocks) for rid in range(3)}
    stats_before = alloc.stats()
    with pytest.raises(RuntimeError, match="out of physical blocks"):
        DecodeBatch(alloc, [0, 1, 2], max_new_tokens=4)
    assert alloc._free_blocks == free_before
    assert {rid: alloc._get_request(rid).logical_blocks for rid in range(3)} == pages_before
    assert alloc.stats() == stats_before
    # the pool still serves a batch that fits
    batch = DecodeBatch(alloc, [0, 1], max_new_tokens=4)
    batch.close()
    assert alloc._free_blocks == free_before
