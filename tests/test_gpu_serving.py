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


def test_decode_batch_attention_bit_identical_to_allocator_cache(monkeypatch):
    """A small batch (32 rows): every step is one fs_paged_decode_append_i8 launch (append is never
    called) and matches the allocator's int64-table cache bit for bit."""

    H, D = 8, 128
    announce("decode batch int32 device table vs allocator int64 table")
    alloc, rids = build_request_pool([300, 17, 1000, 64], heads=H, head_dim=D, headroom_tokens=32, seed=4,
                                     device=DEV)
    batch = DecodeBatch(alloc, rids, max_new_tokens=20, reserve_steps=4)

    def no_separate_append(*_a, **_k):
        raise AssertionError("a one-round grid should take the one-launch step")

    monkeypatch.setattr(DecodeBatch, "append", no_separate_append)
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


@pytest.mark.parametrize("forced_splits,fused", [(None, False), ("4", False), (None, True), ("4", True)])
def test_serving_step_at_scale_b64_ragged_shuffled_pool(monkeypatch, forced_splits, fused):
    """fused: DecodeBatch.step (which takes two launches here: 2048 rows are several rounds of
    workgroups); else append, then attend."""

    B, H, D, bs, steps = 64, 32, 128, 16, 3
    g = torch.Generator().manual_seed(2024)
    lengths = torch.randint(128, 16385, (B,), generator=g).tolist()
    lengths[5] = 16384 - 1  # a request that crosses into a new page on the second step
    lengths[9] = 128        # one exactly at a page boundary: the first append opens a page
    announce(f"serving step B{B} H{H} D{D} ragged [128,16384] sum {sum(lengths)} splits {forced_splits} "
             f"fused {fused}")
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
        if fused:
            out = batch.step(q, kn.to(DEV), vn.to(DEV))
            plain, stats = batch.attend(q, return_stats=True)
            assert torch.equal(out, plain), f"step {step}: fused step vs decode over the appended cache"
        else:
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


def _append_then_decode_reference(cache, kn, vn, lens_in, plan):
    """fs_append_tokens_i8 followed by the paged decode over the advanced lengths (two launches)."""

    lib = _lib.require()
    ks, vs = cache.k_quant, cache.v_quant
    B, H, _, D = kn.shape
    lens_out = torch.empty_like(lens_in)
    dropped = torch.zeros(1, dtype=torch.int32, device=DEV)
    table = cache.block_table
    _lib.check(lib.fs_append_tokens_i8(
        kn.data_ptr(), vn.data_ptr(), _lib.dtype_code(kn.dtype), ks.values.data_ptr(), ks.scale.data_ptr(),
        ks.zero_point.data_ptr(), vs.values.data_ptr(), vs.scale.data_ptr(), vs.zero_point.data_ptr(),
        int(ks.values.shape[0]), table.data_ptr(), table.element_size(), int(table.shape[1]), lens_in.data_ptr(),
        lens_out.data_ptr(), B, H, D, cache.block_size, dropped.data_ptr(), _lib.stream_ptr(DEV)))
    after = fa.PagedKVCache(k_quant=ks, v_quant=vs, block_table=table, lengths=lens_out, block_size=cache.block_size,
                            max_seq_len=plan["max_seq_len"])
    return lens_out, after, int(dropped.item())


def _fused_append_decode(cache, q, kn, vn, lens_in, plan):
    lib = _lib.require()
    from flashspec_amd.triton_utils import MERGE_MAX_WAVES, launch_plan, merge_area

    ks, vs = cache.k_quant, cache.v_quant
    B, H, D = q.shape
    tiled, waves, split_tiles, max_splits, _ = launch_plan(plan["max_seq_len"], B * H, D, cache.block_size,
                                                           cache.block_size, DEV, light=q.dtype == torch.float16)
    assert tiled
    area, area_bytes, ws, ws_bytes = None, 0, None, 0
    if max_splits > 1 and waves <= MERGE_MAX_WAVES:
        area, area_bytes = merge_area(DEV, B * H, max_splits, D)
    elif max_splits > 1:
        ws_bytes = int(lib.fs_decode_workspace_bytes(B * H, max_splits, D))
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=DEV)
    out = torch.empty_like(q)
    lens_out = torch.full_like(lens_in, -7)
    dropped = torch.zeros(1, dtype=torch.int32, device=DEV)
    table = cache.block_table
    _lib.check(lib.fs_paged_decode_append_i8(
        q.data_ptr(), _lib.dtype_code(q.dtype), kn.data_ptr(), vn.data_ptr(), ks.values.data_ptr(),
        ks.scale.data_ptr(), ks.zero_point.data_ptr(), vs.values.data_ptr(), vs.scale.data_ptr(),
        vs.zero_point.data_ptr(), table.data_ptr(), table.element_size(), int(table.shape[1]), lens_in.data_ptr(),
        lens_out.data_ptr(), out.data_ptr(), _lib.ptr(ws), ws_bytes, _lib.ptr(area), area_bytes, B, H, D,
        int(ks.values.shape[0]), cache.block_size, plan["max_seq_len"], 1.0 / float(D) ** 0.5, split_tiles,
        max_splits, waves, dropped.data_ptr(), _lib.stream_ptr(DEV)))
    return out, lens_out, max_splits, waves, split_tiles, int(dropped.item())


def _clone_cache(cache):
    def qt(t):
        return fa.QuantizedTensor(t.values.clone(), t.scale.clone(), t.zero_point.clone(), t.block_size,
                                  t.original_shape)

    return fa.PagedKVCache(k_quant=qt(cache.k_quant), v_quant=qt(cache.v_quant), block_table=cache.block_table.clone(),
                           lengths=cache.lengths.clone(), block_size=cache.block_size, max_seq_len=cache.max_seq_len)


@pytest.mark.parametrize("H,D,qdt,splits,warps,drop", [
    (8, 128, torch.float16, None, None, 250),      # few rows: splits merged in-kernel
    (8, 128, torch.float16, "3", "16", 250),       # 16-wave splits: workspace + merge launch
    # the dropped token's position on a split boundary (15 tiles per split): the decode counts its
    # masked tile as a second split, and the merge launch must count it too
    (8, 128, torch.float16, "3", "16", 240),
    (8, 128, torch.float16, "3", None, 240),       # the same boundary, merged in-kernel
    (32, 128, torch.float16, None, None, 250),     # one split per row
    (8, 64, torch.bfloat16, None, None, 250),
    (4, 256, torch.float32, "2", None, 250),
])
def test_fused_append_decode_bit_identical_to_append_then_decode(monkeypatch, H, D, qdt, splits, warps, drop):
    """fs_paged_decode_append_i8 against fs_append_tokens_i8 + paged decode on a copy of the same
    store: pages, scales, zero points, advanced lengths and outputs bit-identical.  Positions: a
    page's first row (64), its last row (399), mid-page rows (37, 1), the last, part-padded page
    (699), a table entry of -1 at the position (`drop`: token dropped, length kept) and a position
    past the table and max_seq_len (710: likewise)."""

    if splits:
        monkeypatch.setenv("FLASHSPEC_NUM_SPLITS", splits)
    if warps:
        monkeypatch.setenv("FLASHSPEC_NUM_WARPS", warps)
    B, S, bs, max_seq = 7, 700, 16, 704
    announce(f"fused append+decode B{B} H{H} D{D} S{S} q {qdt} splits {splits} warps {warps} drop {drop}")
    k, v = randn((B, H, S, D), 71), randn((B, H, S, D), 72)
    cache = fa.PagedKVCache.from_dense(k.to(DEV), v.to(DEV), block_size=bs, block_table_pattern="shuffled",
                                       layout_seed=3)
    pos = [64, 399, 37, drop, 1, 699, 710]
    table = cache.block_table.clone()
    table[3, drop // bs] = -1
    cache = fa.PagedKVCache(k_quant=cache.k_quant, v_quant=cache.v_quant, block_table=table,
                            lengths=cache.lengths, block_size=bs, max_seq_len=cache.max_seq_len)
    lens_in = torch.tensor(pos, dtype=torch.int64, device=DEV)
    plan = {"max_seq_len": max_seq}
    q = randn((B, H, D), 73, qdt).to(DEV)
    kn, vn = randn((B, H, 1, D), 74, qdt).to(DEV), randn((B, H, 1, D), 75, qdt).to(DEV)
    ref_cache = _clone_cache(cache)
    lens_ref, after, dropped_ref = _append_then_decode_reference(ref_cache, kn, vn, lens_in, plan)
    ref = fa.paged_quant_attention_triton(q, after)
    out, lens_out, max_splits, waves, split_tiles, dropped = _fused_append_decode(cache, q, kn, vn, lens_in, plan)
    torch.cuda.synchronize(DEV)
    announce(f"plan: {max_splits} splits x {waves} waves, {split_tiles} tiles per split")
    if drop == 240:
        assert drop == 16 * split_tiles and max_splits > 1
    assert lens_out.tolist() == lens_ref.tolist() == [65, 400, 38, drop, 2, 700, 710]
    # the two dropped tokens (the -1 entry at `drop`, and 710 past the table / max_seq_len), counted
    # once per request by either path
    assert dropped == dropped_ref == 2
    for ours, theirs, name in ((cache.k_quant, ref_cache.k_quant, "K"), (cache.v_quant, ref_cache.v_quant, "V")):
        assert torch.equal(ours.values, theirs.values), f"{name} values"
        assert torch.equal(ours.scale.view(torch.int32), theirs.scale.view(torch.int32)), f"{name} scales"
        assert torch.equal(ours.zero_point, theirs.zero_point), f"{name} zero points"
    assert torch.equal(out, ref), "fused output vs append + decode"
    # against the oracle on the appended store; request 3 keeps a -1 entry inside its length, which
    # the reference PyTorch path reads as page 0 (the documented divergence), so it is left out
    keep = [0, 1, 2, 4, 5, 6]
    ora = op.OracleCache(from_qt(cache.k_quant), from_qt(cache.v_quant), np_of(table)[keep],
                         np.array(lens_out.tolist(), dtype=np.int64)[keep], bs, max_seq)
    assert_attention_close(out[keep], oa.paged_quant_attention(np_of(q.float())[keep], ora), qdt, "fused vs oracle")


@pytest.mark.parametrize("splits,warps", [(None, None), ("3", None), ("3", "16")])
def test_request_order_gives_the_same_rows(monkeypatch, splits, warps):
    """fs_paged_decode_ordered with the natural order (NULL), reversed, longest-first and random
    permutations: outputs bit-identical to the plain paged decode, for one-split, merged-split and
    workspace-split plans."""

    if splits:
        monkeypatch.setenv("FLASHSPEC_NUM_SPLITS", splits)
    if warps:
        monkeypatch.setenv("FLASHSPEC_NUM_WARPS", warps)
    B, H, S, D = 6, 8, 700, 128
    announce(f"request order B{B} H{H} S{S} splits {splits} warps {warps}")
    k, v = randn((B, H, S, D), 81), randn((B, H, S, D), 82)
    lengths = torch.tensor([700, 5, 333, 0, 640, 17], dtype=torch.int64)
    cache = fa.PagedKVCache.from_dense(k.to(DEV), v.to(DEV), block_size=16, lengths=lengths.to(DEV),
                                       block_table_pattern="shuffled", layout_seed=5)
    q = randn((B, H, D), 83).to(DEV)
    ref = fa.paged_quant_attention_triton(q, cache)
    from flashspec_amd.triton_paged import _run_paged_quant_attention_triton

    g = torch.Generator().manual_seed(1)
    orders = [None, list(range(B))[::-1], sorted(range(B), key=lambda i: -int(lengths[i])),
              torch.randperm(B, generator=g).tolist()]
    for order in orders:
        dev_order = None if order is None else torch.tensor(order, dtype=torch.int32, device=DEV)
        out = _run_paged_quant_attention_triton(q, cache, request_order=dev_order)
        assert torch.equal(out, ref), f"order {order}"


def test_decode_batch_dispatches_longest_first():
    announce("decode batch request order")
    alloc, rids = build_request_pool([300, 17, 1000, 64], heads=4, head_dim=128, headroom_tokens=8, seed=2,
                                     device=DEV)
    batch = DecodeBatch(alloc, rids, max_new_tokens=2)
    assert batch._order.cpu().tolist() == [2, 0, 3, 1]
    q = randn((4, 4, 128), 90).to(DEV)
    assert torch.equal(batch.attend(q), fa.paged_quant_attention_triton(q, alloc.to_cache(rids)))
    batch.close()


@pytest.mark.parametrize("fused", [True, False])
def test_decode_batch_close_raises_when_a_token_was_dropped(fused):
    """A token whose page entry is -1 on the device is dropped by the append (one-launch step or
    append + attend), counted on the device, and close() raises the reference allocator's
    RuntimeError after restoring the free list (reference paged.py:89-90, 222-224)."""

    announce(f"decode batch dropped-token count, fused step {fused}")
    alloc, rids = build_request_pool([48, 70], heads=4, head_dim=128, headroom_tokens=16, seed=5, device=DEV)
    batch = DecodeBatch(alloc, rids, max_new_tokens=3)
    q = randn((2, 4, 128), 91).to(DEV)
    kn, vn = randn((2, 4, 1, 128), 92).to(DEV), randn((2, 4, 1, 128), 93).to(DEV)
    batch.step(q, kn, vn)  # every token finds its page
    assert batch.dropped_tokens() == 0
    pos = batch.host_lengths[0]  # 49: request 0's next token goes to page 3, row 1
    batch.block_table[0, pos // batch.page] = -1
    if fused:
        batch.step(q, kn, vn)
    else:
        batch.append(kn, vn)
        batch.attend(q)
    torch.cuda.synchronize(DEV)
    assert batch.dropped_tokens() == 1
    assert batch.lengths.cpu().tolist() == [pos, batch.host_lengths[1]]  # request 0 kept its length
    with pytest.raises(RuntimeError, match="dropped"):
        batch.close()
    assert not batch._open
    owned = [p for r in rids for p in alloc._get_request(r).logical_blocks]
    assert sorted(alloc._free_blocks + owned) == list(range(alloc.capacity_blocks))  # nothing lost or doubled
