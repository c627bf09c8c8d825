"""GPU parity of the serving pieces: the device-resident decode step (fs_append_tokens_i8 +
paged attention over an int32 device table) against the oracle allocator
(reference src/flashspec/paged.py:108-151, 221-255) and the oracle attention.

Quantized pages are compared bit-exact; attention within max-abs 2e-3 / max-rel 1e-2 (fp16).
The at-scale case (64 ragged requests, lengths in [128, 16384], shuffled pool) checks the
appended pages and the attention of sampled requests against the oracle, and the whole
batch against the allocator's own int64-table cache, bit-identically.
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

import flashspec_amd as fa
from flashspec_amd import _lib
from flashspec_amd.serving import DecodeBatch, ServingConfig, build_request_pool, run_decode_simulation
from oracle import attention as oa
from oracle import paged as op
from oracle import quant as oq
from tests._helpers import assert_attention_close, from_qt, np_of, randn

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


def _assert_stores_equal(alloc, ora, what):
    for ours, ref, name in ((alloc.k_quant, ora.k_quant, "K"), (alloc.v_quant, ora.v_quant, "V")):
        got = from_qt(ours)
        assert np.array_equal(got.values, ref.values), f"{what}: {name} values"
        assert np.array_equal(got.scale.view(np.uint32), ref.scale.view(np.uint32)), f"{what}: {name} scale"
        assert np.array_equal(got.zero_point, ref.zero_point), f"{what}: {name} zero point"


@pytest.mark.parametrize("src_dtype,D", [(torch.float16, 128), (torch.bfloat16, 128), (torch.float32, 128),
                                         (torch.float16, 48), (torch.float32, 64)])
def test_decode_batch_bit_exact_against_oracle_allocator(src_dtype, D):
    """D 128 and 64 take the register-resident append kernel, D 48 the element-wise one."""

    H, bs, cap = 4, 16, 96
    announce(f"decode batch H{H} D{D} page{bs} src {src_dtype}")
    alloc = fa.PagedKVAllocator(capacity_blocks=cap, heads=H, head_dim=D, block_size=bs, device=DEV,
                                dtype=torch.float16)
    ora = op.OracleAllocator(cap, H, D, bs)
    alloc.shuffle_free_blocks(11)
    ora.free = list(alloc._free_blocks)
    for rid, L in enumerate([37, 16, 100, 5, 64]):
        k, v = randn((1, H, L, D), 500 + rid), randn((1, H, L, D), 600 + rid)
        alloc.add_request(rid, k.to(DEV), v.to(DEV))
        ora.add_request(rid, np_of(k.float()), np_of(v.float()))
    alloc.release_request(2)  # its pages come back with stale rows
    ora.release_request(2)
    rids = [0, 1, 3, 4]
    batch = DecodeBatch(alloc, rids, max_new_tokens=40, reserve_steps=8)
    for step in range(40):
        kn = randn((4, H, 1, D), 700 + step, src_dtype)
        vn = randn((4, H, 1, D), 800 + step, src_dtype)
        batch.append(kn.to(DEV), vn.to(DEV))
        ora.append_batch(rids, np_of(kn.float()), np_of(vn.float()))
        if step % 10 == 9:
            torch.cuda.synchronize(DEV)
            _assert_stores_equal(alloc, ora, f"step {step}")
            assert batch.lengths.cpu().tolist() == [ora.requests[r]["length"] for r in rids]
            q = randn((4, H, D), 900 + step)
            got = batch.attend(q.to(DEV))
            assert_attention_close(got, oa.paged_quant_attention(np_of(q), ora.to_cache(rids)), torch.float16,
                                   f"step {step}")
    batch.close()
    assert alloc._free_blocks == ora.free
    for rid in rids:
        assert alloc._requests[rid].logical_blocks == ora.requests[rid]["blocks"]


def test_decode_batch_attention_bit_identical_to_allocator_cache():
    H, D = 8, 128
    announce("decode batch int32 device table vs allocator int64 table")
    alloc, rids = build_request_pool([300, 17, 1000, 64], heads=H, head_dim=D, headroom_tokens=32, seed=4,
                                     device=DEV)
    batch = DecodeBatch(alloc, rids, max_new_tokens=20, reserve_steps=4)
    for step in range(20):
        q = randn((4, H, D), 40 + step).to(DEV)
        kn, vn = randn((4, H, 1, D), 60 + step).to(DEV), randn((4, H, 1, D), 80 + step).to(DEV)
        out = batch.step(q, kn, vn)
        ref = fa.paged_quant_attention_triton(q, alloc.to_cache(rids))
        assert torch.equal(out, ref), f"step {step}"
    batch.close()


def _sub_cache(alloc, pages, length):
    """Oracle cache holding only ``pages`` (one request) of the allocator's store."""

    idx = torch.tensor(pages, dtype=torch.int64, device=DEV)
    H, bs, D = alloc.heads, alloc.block_size, alloc.head_dim

    def sub(q):
        return oq.OracleQuant(np_of(q.values[idx]), np_of(q.scale[idx]), np_of(q.zero_point[idx]), bs,
                              (len(pages), H, bs, D))

    table = np.arange(len(pages), dtype=np.int64)[None, :]
    return op.OracleCache(sub(alloc.k_quant), sub(alloc.v_quant), table, np.array([length], dtype=np.int64), bs,
                          length)


def _page_copy(store, page):
    return (np_of(store.values[page]).copy(), np_of(store.scale[page]).copy(), np_of(store.zero_point[page]).copy())


def _expected_page(before, row, token, H, bs, D):
    """Single-page append (paged.py:121-135): dequantize, replace one row, requantize per head."""

    vals, scale, zero = before
    q = oq.OracleQuant(vals[None], scale[None], zero[None], bs, (1, H, bs, D))
    blk = oq.dequantize_int8_per_block(q).copy()
    blk[0, :, row, :] = token
    return oq.quantize_int8_per_block(blk, bs)


@pytest.mark.parametrize("forced_splits", [None, "4"])
def test_serving_step_at_scale_b64_ragged_shuffled_pool(monkeypatch, forced_splits):
    B, H, D, bs, steps = 64, 32, 128, 16, 3
    g = torch.Generator().manual_seed(2024)
    lengths = torch.randint(128, 16385, (B,), generator=g).tolist()
    lengths[5] = 16384 - 1  # a request that crosses into a new page on the second step
    lengths[9] = 128        # one exactly at a page boundary: the first append opens a page
    announce(f"serving step B{B} H{H} D{D} ragged [128,16384] sum {sum(lengths)} splits {forced_splits}")
    if forced_splits:
        monkeypatch.setenv("FLASHSPEC_NUM_SPLITS", forced_splits)
    alloc, rids = build_request_pool(lengths, heads=H, head_dim=D, headroom_tokens=16, seed=7, device=DEV)
    sample = [5, 9, int(np.argmin(lengths)), int(np.argmax(lengths))]
    batch = DecodeBatch(alloc, rids, max_new_tokens=steps, reserve_steps=2)
    for step in range(steps):
        q = randn((B, H, D), 3000 + step).to(DEV)
        kn, vn = randn((B, H, 1, D), 3100 + step), randn((B, H, 1, D), 3200 + step)
        before = {}
        for i in sample:
            pos = batch.host_lengths[i]
            page = alloc._requests[rids[i]].logical_blocks[pos // bs] if pos // bs < len(
                alloc._requests[rids[i]].logical_blocks) else None
            before[i] = (pos, page)
        pre = {i: (_page_copy(alloc.k_quant, p), _page_copy(alloc.v_quant, p)) for i, (_, p) in before.items()
               if p is not None}
        out, stats = None, None
        batch.append(kn.to(DEV), vn.to(DEV))
        out, stats = batch.attend(q, return_stats=True)
        torch.cuda.synchronize(DEV)
        announce(f"step {step}: num_splits {stats['num_splits']}")
        if forced_splits:
            assert stats["num_splits"] > 1
        for i in sample:
            pos, page = before[i]
            page = alloc._requests[rids[i]].logical_blocks[pos // bs]
            for store, src, k in ((alloc.k_quant, kn, 0), (alloc.v_quant, vn, 1)):
                if i in pre:
                    exp = _expected_page(pre[i][k], pos % bs, np_of(src[i, :, 0].float()), H, bs, D)
                    got = _page_copy(store, page)
                    assert np.array_equal(got[0], exp.values[0]), f"step {step} request {i} page values"
                    assert np.array_equal(got[1].view(np.uint32), exp.scale[0].view(np.uint32))
                    assert np.array_equal(got[2], exp.zero_point[0])
            L = batch.host_lengths[i]
            pages = alloc._requests[rids[i]].logical_blocks[: -(-L // bs)]
            ref = oa.paged_quant_attention(np_of(q[i:i + 1]), _sub_cache(alloc, pages, L))
            assert_attention_close(out[i:i + 1], ref, torch.float16, f"step {step} request {i} (L={L})")
        full = fa.paged_quant_attention_triton(q, alloc.to_cache(rids))
        assert torch.equal(out, full), f"step {step}: int32 device table vs int64 allocator table"
    batch.close()


def test_simulation_uses_device_batch_and_keeps_allocator_consistent():
    announce("serving simulation on GPU with request churn")
    res = run_decode_simulation(ServingConfig(requests=4, prompt_lens=(40, 130), decode_steps=12,
                                              request_life_steps=5, heads=4, head_dim=128, device="cuda",
                                              dtype="float16"))
    assert res["attention_backend"] == "hip"
    assert res["finishes"] == 8 and res["arrivals"] == 12
    assert res["generated_tokens"] == 48
    assert res["used_tokens"] > 0 and 0.0 < res["block_utilization"] <= 1.0
