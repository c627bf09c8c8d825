"""Tree verification host logic on CPU: the portable path against the oracle, validation,
stats keys (flashspec_amd.tree; semantics in oracle/tree.py)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import flashspec_amd as fa
from flashspec_amd.tree import path_mask, tree_shape, validate_parents
from oracle import tree as ot
from tests._helpers import from_cache


def _case(B, H, S, D, N, seed, lengths, page=16, kv_format="affine_block"):
    g = torch.Generator().manual_seed(seed)
    k = torch.randn((B, H, S, D), generator=g)
    v = torch.randn((B, H, S, D), generator=g)
    cache = fa.PagedKVCache.from_dense(k, v, page, lengths=torch.tensor(lengths), block_table_pattern="shuffled",
                                       kv_format=kv_format)
    q = torch.randn((B, N, H, D), generator=g)
    dk = torch.randn((B, N, H, D), generator=g)
    dv = torch.randn((B, N, H, D), generator=g)
    return q, cache, dk, dv


@pytest.mark.parametrize("parents", [[[-1, 0, 1, 2, 3]] * 2, [[-1, -1, 0, 0, 2], [-1, 0, 0, 1, -1]]])
def test_portable_tree_matches_oracle(parents):
    q, cache, dk, dv = _case(2, 3, 37, 16, 5, 3, [37, 9])
    par = torch.tensor(parents)
    got, stats = fa.tree_verify_attention(q, cache, dk, dv, par, return_stats=True)
    ref = ot.tree_verify_attention(q.numpy(), from_cache(cache), dk.numpy(), dv.numpy(), np.array(parents))
    np.testing.assert_allclose(got.numpy(), ref, rtol=1e-5, atol=1e-5)
    assert stats["materializes_dense_kv"] == 1.0 and stats["tree_nodes"] == 5.0
    assert stats["tree_depth"] == float(max(int(m.sum()) for m in ot.path_mask(np.array(parents)).reshape(-1, 5)))


@pytest.mark.parametrize("kv_format", ["fp8_block", "affine_channel", "symmetric_token"])
def test_portable_tree_other_formats(kv_format):
    """The portable path reads every KV format through the cache's own dequantization."""

    parents = [[-1, 0, 0, 1], [-1, -1, 1, 2]]
    q, cache, dk, dv = _case(2, 2, 40, 16, 4, 5, [40, 23], kv_format=kv_format)
    got = fa.tree_verify_attention(q, cache, dk, dv, torch.tensor(parents))
    ref = ot.tree_verify_attention(q.numpy(), from_cache(cache), dk.numpy(), dv.numpy(), np.array(parents))
    np.testing.assert_allclose(got.numpy(), ref, rtol=1e-5, atol=1e-5)


def test_tree_validation():
    q, cache, dk, dv = _case(1, 2, 20, 8, 3, 4, [20])
    for bad in ([[0, -1, -1]], [[-1, 1, 0]], [[-1, 0, 5]], [[-3, -1, 0]]):
        with pytest.raises(ValueError):
            fa.tree_verify_attention(q, cache, dk, dv, torch.tensor(bad))
    with pytest.raises(ValueError):
        fa.tree_verify_attention(q, cache, dk, dv, torch.tensor([[-1, 0]]))
    with pytest.raises(ValueError):
        fa.tree_verify_attention(q[:, :, :1], cache, dk, dv, torch.tensor([[-1, 0, 0]]))
    with pytest.raises(ValueError):
        fa.tree_verify_attention(q, cache, dk, dv, torch.tensor([[-1.0, 0.0, 0.0]]))
    assert validate_parents(torch.tensor([[-1, 0, 1]], dtype=torch.int32), 1, 3).dtype == torch.int64
    assert path_mask(torch.tensor([[-1, 0, 0, 2]]))[0].tolist() == ot.path_mask(np.array([[-1, 0, 0, 2]]))[0].tolist()
    # validate=False only skips the check for parents already on the GPU: CPU calls still check
    with pytest.raises(ValueError):
        fa.tree_verify_attention(q, cache, dk, dv, torch.tensor([[-1, 0, 5]]), validate=False)



def test_tree_shape_counts():
    # request 0: root children {0, 4}, node 0 -> {1, 2}, 1 -> {3}, 4 -> {5}: leaves 2, 3, 5
    # request 1: a chain of 6
    shape = tree_shape(torch.tensor([[-1, 0, 0, 1, -1, 4], [-1, 0, 1, 2, 3, 4]]))
    assert shape == {"depth": 6, "leaves": 3, "max_branch": 2}
    assert tree_shape(torch.tensor([[-1, -1, -1]])) == {"depth": 1, "leaves": 3, "max_branch": 3}


def test_parents_cache_hit_on_another_stream_records_that_stream():
    """A cached parents copy reused on a second stream waits for the copy and is registered with
    the caching allocator for that stream (record_stream); on its own stream neither happens."""

    from flashspec_amd.tree import _reuse_on

    class Stream:
        def __init__(self, name):
            self.name, self.waited = name, []

        def wait_event(self, ev):
            self.waited.append(ev)

    class Tensor:
        def __init__(self):
            self.recorded = []

        def record_stream(self, s):
            self.recorded.append(s)

    made_on, other, ready, t = Stream("made"), Stream("other"), object(), Tensor()
    assert _reuse_on((t, made_on, ready), made_on) is t
    assert t.recorded == [] and made_on.waited == []
    assert _reuse_on((t, made_on, ready), other) is t
    assert other.waited == [ready] and t.recorded == [other]
