"""In-kernel split merge (fs_fused_decode_merged / fs_paged_decode_merged): rows split across
workgroups and the last split of each row to finish merges it inside the decode launch.

Checked on the GPU against the oracle and against the two-launch path (split partials in a
workspace + fs_combine_splits), for every KV format the tiled kernel serves, ragged and empty
rows, many split counts in a row on one merge area (which every launch must leave all zero), and
graph capture with replays."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import flashspec_amd as fa
from flashspec_amd import _lib, triton_utils
from oracle import attention as oa
from oracle import quant as oq
from tests._helpers import assert_attention_close, np_of, oracle_paged_attention, randn

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)


@pytest.fixture(autouse=True)
def _clean_env(monkeypatch):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    for key in ("FLASHSPEC_NUM_SPLITS", "FLASHSPEC_BLOCK_N", "FLASHSPEC_NUM_WARPS"):
        monkeypatch.delenv(key, raising=False)


def announce(msg: str) -> None:
    print(f"[gpu case] {msg}", flush=True)


def _area_is_zero() -> bool:
    torch.cuda.synchronize(DEV)
    stream = torch.cuda.current_stream(DEV)
    area = triton_utils._MERGE_AREAS.get((DEV.index, stream.cuda_stream))
    return area is not None and int(area.count_nonzero().item()) == 0


def _paged(B, H, S, D, seed, lengths, kv_format="affine_block", layout="shuffled", page=16):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn((B, H, D), generator=g).to(torch.float16)
    k = torch.randn((B, H, S, D), generator=g).to(torch.float16)
    v = torch.randn((B, H, S, D), generator=g).to(torch.float16)
    cache = fa.PagedKVCache.from_dense(k.to(DEV), v.to(DEV), block_size=page, lengths=torch.tensor(lengths).to(DEV),
                                       block_table_pattern=layout, layout_seed=seed, kv_format=kv_format)
    return q, cache


@pytest.mark.parametrize("kv_format", ["affine_block", "symmetric_token", "fp8_block", "affine_channel"])
def test_paged_split_merge_matches_oracle_and_two_launch_path(monkeypatch, kv_format):
    """Forced splits 2..16 over one merge area: each launch within tolerance of the oracle, of the
    two-launch combine path, and the area all zero afterwards."""

    page = 32 if kv_format == "affine_channel" else 16
    q, cache = _paged(3, 8, 1111, 128, 21, [1111, 640, 0], kv_format=kv_format, page=page)
    qd = q.to(DEV)
    ref = oracle_paged_attention(q, cache)
    for splits in (2, 3, 5, 8, 16):
        announce(f"paged {kv_format} merged split {splits}")
        monkeypatch.setenv("FLASHSPEC_NUM_SPLITS", str(splits))
        got, st = fa.paged_quant_attention_triton(qd, cache, return_stats=True)
        assert st["tiled_path"] == 1.0 and st["num_splits"] > 1
        assert _area_is_zero(), f"merge area not left zero after {splits} splits"
        # the empty row (length 0) writes zeros, as the Triton kernels do
        assert torch.count_nonzero(got[2]).item() == 0
        assert_attention_close(got[:2], ref[:2], torch.float16, f"{kv_format} splits {splits}")


@pytest.mark.parametrize("layout", ["contiguous", "interleaved"])
def test_paged_split_merge_equals_combine_launch(monkeypatch, layout):
    """The same split plan through fs_paged_decode_i8 + fs_combine_splits (partials in a torch
    workspace): the two merges agree to fp32 rounding."""

    q, cache = _paged(4, 32, 2048, 128, 22, [2048, 2000, 1024, 17], layout=layout)
    qd = q.to(DEV)
    monkeypatch.setenv("FLASHSPEC_NUM_SPLITS", "4")
    got, st = fa.paged_quant_attention_triton(qd, cache, return_stats=True)
    split_tiles, max_splits, waves = int(st["split_tiles"]), int(st["num_splits"]), int(st["num_warps"])
    lib = _lib.require()
    kq, vq = cache.k_quant, cache.v_quant
    wsb = int(lib.fs_decode_workspace_bytes(4 * 32, max_splits, 128))
    ws = torch.empty(wsb, dtype=torch.uint8, device=DEV)
    two = torch.empty_like(qd)
    stream = _lib.stream_ptr(DEV)
    _lib.check(lib.fs_paged_decode_i8(
        qd.data_ptr(), 1, *(t.data_ptr() for t in (kq.values, kq.scale, kq.zero_point, vq.values, vq.scale,
                                                    vq.zero_point)),
        cache.block_table.data_ptr(), 8, int(cache.block_table.shape[1]), cache.lengths.data_ptr(), two.data_ptr(),
        ws.data_ptr(), wsb, 4, 32, 128, int(kq.original_shape[0]), 16, 16, 2048, 1 / math.sqrt(128), split_tiles,
        max_splits, waves, stream))
    _lib.check(lib.fs_combine_splits(ws.data_ptr(), cache.lengths.data_ptr(), two.data_ptr(), 1, 4, 32, 128, 2048,
                                     split_tiles, max_splits, stream))
    torch.cuda.synchronize(DEV)
    assert (got.float() - two.float()).abs().max().item() <= 1e-3
    assert_attention_close(got, oracle_paged_attention(q, cache), torch.float16, "merged vs oracle")


@pytest.mark.parametrize("q_dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_fused_split_merge_half_empty_grid(monkeypatch, q_dtype):
    """Contiguous rows with the automatic plan and with forced splits, every query dtype."""

    B, H, S, D = 4, 32, 2048, 128
    q = randn((B, H, D), 31, q_dtype)
    k = randn((B, H, S, D), 32)
    v = randn((B, H, S, D), 33)
    kq, vq = oq.quantize_int8_per_block(np_of(k.float()), 16), oq.quantize_int8_per_block(np_of(v.float()), 16)
    lens = torch.tensor([2048, 1500, 33, 2047])
    ref = oa.fused_dequant_attention(np_of(q.float()), kq, vq, np_of(lens))
    kd = fa.quantize_int8_per_block(k.to(DEV), 16)
    vd = fa.quantize_int8_per_block(v.to(DEV), 16)
    for forced in (None, "2", "4", "7"):
        if forced is None:
            monkeypatch.delenv("FLASHSPEC_NUM_SPLITS", raising=False)
        else:
            monkeypatch.setenv("FLASHSPEC_NUM_SPLITS", forced)
        announce(f"fused merged {q_dtype} splits {forced}")
        got = fa.fused_dequant_attention_triton(q.to(DEV), kd, vd, lengths=lens.to(DEV))
        assert _area_is_zero()
        assert_attention_close(got, ref, q_dtype, f"splits {forced}")


@pytest.mark.parametrize("B,S,splits", [(2, 8192, 8), (1, 16384, 8), (4, 2048, 2)])
def test_split_merge_sixteen_wave_workgroups(B, S, splits):
    """fs_paged_decode_merged with 16-wave workgroups (1024 threads; the Python launcher keeps
    the two-launch path for them, which is faster there): the last split's waves finish their
    reads at different times, and no word may be cleared before all of them have read it (no NaN,
    oracle agreement, area zero, bit-identical repeats)."""

    q, cache = _paged(B, 32, S, 128, 24, [S] * B, layout="contiguous")
    qd = q.to(DEV)
    ref = oracle_paged_attention(q, cache)
    lib = _lib.require()
    rows, tiles = B * 32, S // 16
    split_tiles = math.ceil(tiles / splits)
    max_splits = math.ceil(tiles / split_tiles)
    area, area_bytes = triton_utils.merge_area(DEV, rows, max_splits, 128)
    kq, vq = cache.k_quant, cache.v_quant
    first = None
    for rep in range(5):
        announce(f"16-wave merge B{B} S{S} splits {max_splits} rep {rep}")
        got = torch.empty_like(qd)
        _lib.check(lib.fs_paged_decode_merged(
            qd.data_ptr(), 1, 0, *(t.data_ptr() for t in (kq.values, kq.scale, kq.zero_point, vq.values, vq.scale,
                                                           vq.zero_point)),
            cache.block_table.data_ptr(), 8, int(cache.block_table.shape[1]), cache.lengths.data_ptr(),
            got.data_ptr(), area.data_ptr(), area_bytes, B, 32, 128, int(kq.original_shape[0]), 16, 16, S,
            1 / math.sqrt(128), split_tiles, max_splits, 16, _lib.stream_ptr(DEV)))
        torch.cuda.synchronize(DEV)
        assert not torch.isnan(got).any(), f"rep {rep}: NaN rows (a merge wait ran out)"
        assert _area_is_zero()
        if first is None:
            first = got
            assert_attention_close(got, ref, torch.float16, "16-wave merge")
        else:
            assert torch.equal(got, first), f"rep {rep} not bit-identical"


def test_launcher_keeps_two_launch_path_for_sixteen_waves(monkeypatch):
    """Forced 16-wave split plans go through the workspace + merge launch (faster there) and agree
    with the oracle."""

    monkeypatch.setenv("FLASHSPEC_NUM_SPLITS", "8")
    monkeypatch.setenv("FLASHSPEC_NUM_WARPS", "16")
    q, cache = _paged(2, 32, 8192, 128, 25, [8192, 5000], layout="contiguous")
    got, st = fa.paged_quant_attention_triton(q.to(DEV), cache, return_stats=True)
    torch.cuda.synchronize(DEV)
    assert st["num_warps"] == 16.0 and st["num_splits"] == 8.0
    assert_attention_close(got, oracle_paged_attention(q, cache), torch.float16, "16-wave two-launch")


def test_graph_replay_with_split_merge(monkeypatch):
    """A captured split decode zero-fills its own merge area inside the graph: every replay,
    with eager split decodes on the same stream between replays, equals the eager result."""

    monkeypatch.setenv("FLASHSPEC_NUM_SPLITS", "4")
    q, cache = _paged(2, 16, 777, 128, 23, [777, 300])
    qd = q.to(DEV)
    eager = fa.paged_quant_attention_triton(qd, cache)
    torch.cuda.synchronize(DEV)
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
        torch.cuda.synchronize(DEV)
        again = fa.paged_quant_attention_triton(qd, cache)  # eager split decode between replays
        torch.cuda.synchronize(DEV)
        assert torch.equal(out, eager), f"replay {i}"
        assert torch.equal(again, eager), f"eager after replay {i}"


def test_stale_merge_words_from_earlier_launches_are_not_taken(monkeypatch):
    """Every word of the merge area planted with a stale tag and a value far off the result: the
    next split decode reads past them (each launch tags its words with a fresh value; a plain
    tag of 1 is what every word carried before per-launch tags), overwrites and clears them, and
    gives the same bits as before the planting."""

    import struct

    monkeypatch.setenv("FLASHSPEC_NUM_SPLITS", "4")
    B, H, D = 2, 8, 128
    q, cache = _paged(B, H, 1000, D, 24, [1000, 777])
    qd = q.to(DEV)
    first, st = fa.paged_quant_attention_triton(qd, cache, return_stats=True)
    assert st["num_splits"] == 4.0 and st["num_warps"] <= triton_utils.MERGE_MAX_WAVES  # in-launch merge
    assert _area_is_zero()
    area = triton_utils._MERGE_AREAS[(DEV.index, _lib.stream_ptr(DEV))]
    rows, splits = B * H, int(st["num_splits"])
    counts = (rows * 4 + 255) // 256 * 256
    slots = area[counts:counts + rows * splits * (D + 2) * 8].view(torch.int64)
    stale = (1 << 32) | struct.unpack("<I", struct.pack("<f", 1e30))[0]
    try:
        announce("stale tagged words in the merge area")
        slots.fill_(stale)
        torch.cuda.synchronize(DEV)
        again = fa.paged_quant_attention_triton(qd, cache)
        assert _area_is_zero(), "the launch left planted words behind"
        assert torch.equal(again, first)
        assert_attention_close(again, oracle_paged_attention(q, cache), torch.float16, "after stale words")
    finally:
        area.zero_()
        torch.cuda.synchronize(DEV)
