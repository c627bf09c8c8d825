"""fs_paged_decode_i8_noalloc (split-K partials in the library's per-GPU device array) against
fs_paged_decode_i8 + fs_combine_splits with a torch workspace, through the C ABI: bit-identical
outputs on two calls in a row, the second smaller, plus a one-split call; both checked against the
oracle.  Collected last so that a failure here cannot hide other tests."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import flashspec_amd as fa
from flashspec_amd import _lib
from tests._helpers import assert_attention_close, oracle_paged_attention

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0)


def _case(B, H, S, D, seed, lengths):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn((B, H, D), generator=g).to(torch.float16)
    k = torch.randn((B, H, S, D), generator=g).to(torch.float16)
    v = torch.randn((B, H, S, D), generator=g).to(torch.float16)
    cache = fa.PagedKVCache.from_dense(k.to(DEV), v.to(DEV), block_size=16, lengths=torch.tensor(lengths).to(DEV),
                                       block_table_pattern="shuffled", layout_seed=seed)
    return q, cache


def _args(q, cache):
    kq, vq = cache.k_quant, cache.v_quant
    B, H, D = q.shape
    return dict(q=q.data_ptr(), kv=[t.data_ptr() for t in (kq.values, kq.scale, kq.zero_point, vq.values, vq.scale,
                                                           vq.zero_point)],
                table=cache.block_table, lengths=cache.lengths, B=B, H=H, D=D,
                pages=int(kq.original_shape[0]), S=int(cache.max_seq_len))


def _with_workspace(lib, a, out, split_tiles, max_splits, waves, stream):
    ws_bytes = int(lib.fs_decode_workspace_bytes(a["B"] * a["H"], max_splits, a["D"]))
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=DEV)
    _lib.check(lib.fs_paged_decode_i8(a["q"], 1, *a["kv"], a["table"].data_ptr(), 8, int(a["table"].shape[1]),
                                      a["lengths"].data_ptr(), out.data_ptr(), ws.data_ptr(), ws_bytes, a["B"], a["H"],
                                      a["D"], a["pages"], 16, 16, a["S"], 1.0 / math.sqrt(a["D"]), split_tiles,
                                      max_splits, waves, stream))
    if max_splits > 1:
        _lib.check(lib.fs_combine_splits(ws.data_ptr(), a["lengths"].data_ptr(), out.data_ptr(), 1, a["B"], a["H"],
                                         a["D"], a["S"], split_tiles, max_splits, stream))
    return ws


def _no_alloc(lib, a, out, split_tiles, max_splits, waves, stream):
    _lib.check(lib.fs_paged_decode_i8_noalloc(a["q"], 1, *a["kv"], a["table"].data_ptr(), 8,
                                              int(a["table"].shape[1]), a["lengths"].data_ptr(), out.data_ptr(),
                                              a["B"], a["H"], a["D"], a["pages"], 16, 16, a["S"],
                                              1.0 / math.sqrt(a["D"]), split_tiles, max_splits, waves, stream))


@pytest.mark.parametrize("plan_first,plan_second", [((8, 4), (4, 2)), ((16, 8), (8, 2))])
def test_no_alloc_matches_workspace_entry_point_twice(plan_first, plan_second):
    """Two calls in a row on the shared device array (the second over a smaller batch and a
    shorter sequence); each bit-identical to the workspace entry point and within tolerance of
    the oracle."""

    lib = _lib.require()
    stream = _lib.stream_ptr(DEV)
    cases = [(_case(4, 8, 1000, 128, 3, [1000, 777, 16, 1]), plan_first),
             (_case(2, 8, 300, 128, 4, [300, 129]), plan_second)]
    for (q, cache), (split_tiles, waves) in cases:
        qd = q.to(DEV)
        a = _args(qd, cache)
        max_splits = math.ceil(math.ceil(a["S"] / 16) / split_tiles)
        print(f"no-alloc B{a['B']} S{a['S']} split_tiles {split_tiles} splits {max_splits} waves {waves}",
              flush=True)
        ref = torch.empty_like(qd)
        got = torch.full_like(qd, float("nan"))
        ws = _with_workspace(lib, a, ref, split_tiles, max_splits, waves, stream)
        _no_alloc(lib, a, got, split_tiles, max_splits, waves, stream)
        torch.cuda.synchronize(DEV)
        del ws
        assert max_splits > 1
        assert torch.equal(got, ref)
        assert_attention_close(got, oracle_paged_attention(q, cache), torch.float16, "no-alloc")


def test_no_alloc_one_split_and_size_limit():
    """One split needs no scratch (the decode writes the output); a plan whose partials exceed the
    array is rejected before any launch."""

    lib = _lib.require()
    stream = _lib.stream_ptr(DEV)
    q, cache = _case(2, 4, 200, 64, 5, [200, 57])
    qd = q.to(DEV)
    a = _args(qd, cache)
    ref, got = torch.empty_like(qd), torch.full_like(qd, float("nan"))
    _with_workspace(lib, a, ref, 13, 1, 2, stream)
    _no_alloc(lib, a, got, 13, 1, 2, stream)
    torch.cuda.synchronize(DEV)
    assert torch.equal(got, ref)
    limit = int(lib.fs_noalloc_scratch_bytes())
    assert limit == 16 << 20
    # 256 rows x 1024 splits x (128 + 2) floats > 16 MiB
    rc = lib.fs_paged_decode_i8_noalloc(a["q"], 1, *a["kv"], a["table"].data_ptr(), 8, int(a["table"].shape[1]),
                                        a["lengths"].data_ptr(), got.data_ptr(), 8, 32, 128, a["pages"], 16, 16,
                                        16384, 0.1, 1, 1024, 1, stream)
    assert rc == _lib.FS_ERR_INVALID and "at most" in lib.fs_last_error().decode()
