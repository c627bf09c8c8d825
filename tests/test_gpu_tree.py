"""GPU parity of tree verification (fs_tree_verify_i8) against the oracle (oracle/tree.py).

Attention within max-abs 2e-3 / max-rel 1e-2 (fp16 outputs).  Cases cover chains (which
reduce to paged decode over prefix + path), stars, random forests, empty prefixes, the
shuffled page layout, 8-token and per-token quantization, head dims 64/96/128/256, and the
prefix partials of rows that split.
"""

from __future__ import annotations

import sys

import numpy as np
import pytest
import torch

import flashspec_amd as fa
from flashspec_amd import _lib
from oracle import tree as ot
from tests._helpers import assert_attention_close, from_cache, np_of, randn

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
    for key in ("FLASHSPEC_NUM_SPLITS", "FLASHSPEC_BLOCK_N", "FLASHSPEC_NUM_WARPS", "FLASHSPEC_TREE_NODES_PER_WG"):
        monkeypatch.delenv(key, raising=False)


def _random_parents(B, N, seed):
    rng = np.random.default_rng(seed)
    par = np.full((B, N), -1, dtype=np.int64)
    for b in range(B):
        for n in range(1, N):
            par[b, n] = rng.integers(-1, n)
    return par


def _run(B, H, S, D, N, parents, lengths, page=16, layout="shuffled", q_dtype=torch.float16, kv_format="affine_block",
         seed=0, kernel="auto", q_scale=1.0, draft_dtype=torch.float16):
    q = (randn((B, N, H, D), seed + 1, torch.float32) * q_scale).to(q_dtype)
    k = randn((B, H, S, D), seed + 2)
    v = randn((B, H, S, D), seed + 3)
    dk = randn((B, N, H, D), seed + 4, torch.float32).to(draft_dtype)
    dv = randn((B, N, H, D), seed + 5, torch.float32).to(draft_dtype)
    cache = fa.PagedKVCache.from_dense(k.to(DEV), v.to(DEV), page, lengths=torch.tensor(lengths).to(DEV),
                                       block_table_pattern=layout, layout_seed=seed, kv_format=kv_format)
    got, stats = fa.tree_verify_attention(q.to(DEV), cache, dk.to(DEV), dv.to(DEV),
                                          torch.tensor(parents).to(DEV), return_stats=True, kernel=kernel)
    torch.cuda.synchronize(DEV)
    ref = ot.tree_verify_attention(np_of(q.float()), from_cache(cache), np_of(dk.float()), np_of(dv.float()),
                                   np.asarray(parents))
    return got, ref, stats


@pytest.mark.parametrize("B,H,S,D,N,kind,lengths", [
    (2, 4, 300, 128, 6, "chain", [300, 77]),
    (2, 4, 300, 128, 6, "star", [300, 77]),
    (3, 8, 513, 128, 8, "random", [513, 1, 200]),
    (2, 2, 129, 64, 5, "random", [129, 0]),        # an empty prefix
    (1, 4, 700, 256, 4, "random", [700]),
    (2, 3, 90, 96, 7, "random", [90, 45]),
])
@pytest.mark.parametrize("kernel", ["auto", "rows"])
def test_tree_verify_matches_oracle(B, H, S, D, N, kind, lengths, kernel):
    announce(f"tree verify B{B} H{H} S{S} D{D} N{N} {kind} lengths={lengths} kernel={kernel}")
    if kind == "chain":
        parents = np.tile(np.arange(-1, N - 1), (B, 1))
    elif kind == "star":
        parents = np.full((B, N), -1)
    else:
        parents = _random_parents(B, N, S + N)
    got, ref, stats = _run(B, H, S, D, N, parents, lengths, seed=B + S, kernel=kernel)
    assert stats["materializes_dense_kv"] == 0.0
    assert stats["mfma_prefix"] == float(kernel == "auto" and D in (64, 128, 256))
    assert_attention_close(got.reshape(B * N, H, D), ref.reshape(B * N, H, D), torch.float16, f"tree {kind}")


@pytest.mark.parametrize("page,kv_format,q_dtype", [(8, "affine_block", torch.float16),
                                                    (16, "symmetric_token", torch.bfloat16),
                                                    (32, "affine_block", torch.float32),
                                                    (16, "fp8_block", torch.float16),
                                                    (32, "fp8_block", torch.bfloat16),
                                                    (16, "affine_channel", torch.float16),
                                                    (64, "affine_channel", torch.float32)])
def test_tree_verify_formats(page, kv_format, q_dtype):
    announce(f"tree verify page{page} {kv_format} {q_dtype}")
    B, H, S, D, N = 2, 4, 260, 128, 6
    parents = _random_parents(B, N, page)
    got, ref, stats = _run(B, H, S, D, N, parents, [260, 100], page=page, kv_format=kv_format, q_dtype=q_dtype)
    # FP8 and per-channel stores run the row-kernel prefix (the multi-query kernel reads INT8
    # block / token parameters)
    assert stats["mfma_prefix"] == float(kv_format != "affine_channel" and page % 16 == 0)
    assert_attention_close(got.reshape(B * N, H, D), ref.reshape(B * N, H, D), q_dtype, kv_format)


@pytest.mark.parametrize("D,N", [(128, 12), (64, 40)])
def test_tree_mfma_fp8_per_token(D, N):
    """FP8 codes with one scale per token (token mode of the multi-query kernel, no zero points)."""

    announce(f"tree mfma fp8 per token D{D} N{N}")
    B, H, S, page = 2, 4, 333, 16
    k, v = randn((B, H, S, D), 81).to(DEV), randn((B, H, S, D), 82).to(DEV)
    nbps = -(-S // page)
    pk = fa.PagedKVCache._physical_pages(k, page, None)
    pv = fa.PagedKVCache._physical_pages(v, page, None)
    lens = torch.tensor([S, 150], dtype=torch.int64, device=DEV)
    cache = fa.PagedKVCache(k_quant=fa.quantize_fp8_per_block(pk, 1), v_quant=fa.quantize_fp8_per_block(pv, 1),
                            block_table=torch.arange(B * nbps, dtype=torch.int64, device=DEV).reshape(B, nbps),
                            lengths=lens, block_size=page, max_seq_len=S)
    parents = _random_parents(B, N, 11)
    q = randn((B, N, H, D), 83).to(DEV)
    dk, dv = randn((B, N, H, D), 84).to(DEV), randn((B, N, H, D), 85).to(DEV)
    got, stats = fa.tree_verify_attention(q, cache, dk, dv, torch.tensor(parents), return_stats=True, kernel="mfma")
    torch.cuda.synchronize(DEV)
    assert stats["mfma_prefix"] == 1.0
    ref = ot.tree_verify_attention(np_of(q.cpu().float()), from_cache(cache), np_of(dk.cpu().float()),
                                   np_of(dv.cpu().float()), parents)
    assert_attention_close(got.reshape(B * N, H, D), ref.reshape(B * N, H, D), torch.float16, "fp8 per token")


def test_tree_mfma_rejects_per_channel():
    announce("tree mfma rejects affine_channel")
    B, H, S, D, N = 1, 2, 64, 64, 3
    with pytest.raises(ValueError):
        _run(B, H, S, D, N, [[-1, 0, 0]], [64], kv_format="affine_channel", kernel="mfma")


def test_tree_verify_split_rows(monkeypatch):
    """Prefix rows that split (forced 4 splits) merge their partials in the tail kernel."""

    announce("tree verify with forced split-K")
    monkeypatch.setenv("FLASHSPEC_NUM_SPLITS", "4")
    B, H, S, D, N = 1, 2, 2048, 128, 5
    parents = np.array([[-1, 0, 1, 0, 3]])
    got, ref, stats = _run(B, H, S, D, N, parents, [2048], seed=9)
    assert stats["num_splits"] == 4.0
    assert_attention_close(got.reshape(B * N, H, D), ref.reshape(B * N, H, D), torch.float16, "split")


def test_tree_single_node_matches_paged_decode_plus_token():
    """One root node: the tree output equals paged decode over the prefix extended by the
    node's own token, computed by the oracle as plain attention over concatenated K/V."""

    announce("tree verify single node")
    B, H, S, D = 2, 4, 200, 128
    got, ref, _ = _run(B, H, S, D, 1, np.full((B, 1), -1), [200, 64], seed=21)
    assert_attention_close(got.reshape(B, H, D), ref.reshape(B, H, D), torch.float16, "single node")


def test_tree_device_parents_without_validation():
    """validate=False with parents on the GPU: a valid tree gives the validated result; a parent
    outside [-1, n) ends that node's path there (the oracle sees the tree with it set to -1)."""

    announce("tree verify device parents, validate=False")
    B, H, S, D, N = 2, 4, 160, 128, 6
    q = randn((B, N, H, D), 31).to(DEV)
    k, v = randn((B, H, S, D), 32).to(DEV), randn((B, H, S, D), 33).to(DEV)
    dk, dv = randn((B, N, H, D), 34).to(DEV), randn((B, N, H, D), 35).to(DEV)
    cache = fa.PagedKVCache.from_dense(k, v, 16, block_table_pattern="shuffled", layout_seed=3)
    good = np.array([[-1, 0, 1, 1, -1, 4], [-1, -1, 0, 2, 3, 0]])
    a = fa.tree_verify_attention(q, cache, dk, dv, torch.tensor(good, dtype=torch.int32))
    b = fa.tree_verify_attention(q, cache, dk, dv, torch.tensor(good).to(DEV), validate=False)
    torch.cuda.synchronize(DEV)
    assert torch.equal(a, b)
    bad = good.copy()
    bad[0, 3], bad[1, 5] = 7, -5  # a forward edge and an out-of-range parent
    got = fa.tree_verify_attention(q, cache, dk, dv, torch.tensor(bad).to(DEV), validate=False)
    torch.cuda.synchronize(DEV)
    cut = good.copy()
    cut[0, 3], cut[1, 5] = -1, -1
    ref = ot.tree_verify_attention(np_of(q.cpu().float()), from_cache(cache), np_of(dk.cpu().float()),
                                   np_of(dv.cpu().float()), cut)
    assert_attention_close(got.reshape(B * N, H, D), ref.reshape(B * N, H, D), torch.float16, "cut tree")


# Multi-query MFMA prefix kernel: (B, H, S, D, N, page, kv_format, q dtype, lengths)
MFMA_CASES = [
    (2, 8, 1000, 128, 16, 16, "affine_block", torch.float16, [1000, 333]),
    (1, 4, 700, 128, 17, 32, "affine_block", torch.float16, [700]),          # two node groups, 32-token pages
    (2, 2, 257, 64, 40, 16, "symmetric_token", torch.bfloat16, [257, 16]),  # three groups, per-token scales
    (1, 4, 530, 256, 9, 16, "affine_block", torch.float32, [530]),
    (2, 4, 100, 128, 5, 64, "affine_block", torch.bfloat16, [100, 0]),      # 64-token pages, an empty prefix
    (3, 8, 2100, 128, 12, 16, "symmetric_token", torch.float16, [2100, 5, 1500]),
    (2, 4, 333, 256, 3, 32, "symmetric_token", torch.float16, [333, 200]),
    (1, 16, 4096, 64, 16, 16, "affine_block", torch.float32, [4096]),
    (1, 2, 200, 64, 70, 16, "affine_block", torch.float16, [200]),          # > 64 nodes: tail walks memory
    (2, 4, 1500, 128, 33, 16, "affine_block", torch.bfloat16, [1500, 900]),
    (2, 4, 600, 128, 16, 16, "fp8_block", torch.float16, [600, 250]),         # FP8 codes as fp16 operands
    (1, 4, 300, 64, 20, 32, "fp8_block", torch.bfloat16, [300]),
    (2, 2, 400, 256, 6, 16, "fp8_block", torch.float32, [400, 7]),
    # 512 workgroups of 32 nodes: more than one per CU, so the waves pace each other; drafts staged in LDS
    (8, 32, 256, 128, 64, 16, "affine_block", torch.float16, [256, 256, 100, 256, 17, 256, 256, 240]),
    # fp16 drafts as MFMA tile pairs in split 0 of rows that split, and with an empty prefix
    (2, 4, 3000, 128, 48, 16, "affine_block", torch.float16, [3000, 0]),
    (1, 4, 900, 64, 40, 16, "affine_block", torch.float16, [900]),          # head_dim 64: V rows in halves
]


@pytest.mark.parametrize("B,H,S,D,N,page,fmt,q_dtype,lengths", MFMA_CASES)
def test_tree_mfma_prefix_matches_oracle(B, H, S, D, N, page, fmt, q_dtype, lengths):
    announce(f"tree mfma B{B} H{H} S{S} D{D} N{N} page{page} {fmt} {q_dtype} lengths={lengths}")
    parents = _random_parents(B, N, S + 7 * N)
    got, ref, stats = _run(B, H, S, D, N, parents, lengths, page=page, kv_format=fmt, q_dtype=q_dtype,
                           seed=S + N, kernel="mfma")
    assert stats["mfma_prefix"] == 1.0
    assert_attention_close(got.reshape(B * N, H, D), ref.reshape(B * N, H, D), q_dtype, f"mfma {fmt}")


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("kernel", ["mfma", "rows"])
def test_tree_one_hot_rows_at_extreme_logits(D, kernel):
    """fp32 queries scaled by 1e20: every row's softmax is one-hot over its prefix and path tokens,
    which holds only where exp2(score - max) sees the same rounded score as the running max (the
    MFMA prefix kernel, the path walks, and the decode rows of kernel="rows")."""

    announce(f"tree one-hot rows D{D} kernel={kernel}")
    B, H, S, N = 2, 4, 300, 6
    parents = _random_parents(B, N, 9)
    got, ref, _ = _run(B, H, S, D, N, parents, [300, 150], q_dtype=torch.float32, seed=43, kernel=kernel,
                       q_scale=1e20)
    assert_attention_close(got.reshape(B * N, H, D), ref.reshape(B * N, H, D), torch.float32, "one-hot rows")


@pytest.mark.parametrize("q_dtype,q_scale", [(torch.bfloat16, 3000.0), (torch.bfloat16, 1e-3), (torch.float32, 40.0),
                                             (torch.float32, 1e-4), (torch.float16, 20.0)])
def test_tree_mfma_query_magnitudes(q_dtype, q_scale):
    """Queries far from unit scale: the per-node power-of-two scaling keeps bf16 / fp32 queries
    exact (bf16) or hi+lo exact to ~22 bits (fp32) in the fp16 operands; a large-magnitude fp16
    query makes the softmax nearly one-hot."""

    announce(f"tree mfma q magnitude {q_dtype} x{q_scale}")
    B, H, S, D, N = 2, 4, 300, 128, 6
    parents = _random_parents(B, N, 5)
    got, ref, _ = _run(B, H, S, D, N, parents, [300, 150], q_dtype=q_dtype, seed=41, kernel="mfma", q_scale=q_scale)
    assert_attention_close(got.reshape(B * N, H, D), ref.reshape(B * N, H, D), q_dtype, "q magnitude")


@pytest.mark.parametrize("splits,warps", [("3", "2"), ("1", "1"), ("7", "8")])
def test_tree_mfma_forced_plans(monkeypatch, splits, warps):
    """Split counts and workgroup sizes away from the default plan (the LDS merge of 1..8 waves,
    split partials merged by the tail kernel)."""

    announce(f"tree mfma forced splits={splits} warps={warps}")
    monkeypatch.setenv("FLASHSPEC_NUM_SPLITS", splits)
    monkeypatch.setenv("FLASHSPEC_NUM_WARPS", warps)
    monkeypatch.setenv("FLASHSPEC_BLOCK_N", "16")
    B, H, S, D, N = 2, 4, 1500, 128, 10
    parents = _random_parents(B, N, 8)
    got, ref, stats = _run(B, H, S, D, N, parents, [1500, 700], seed=43, kernel="mfma")
    assert stats["num_warps"] == float(warps)
    assert_attention_close(got.reshape(B * N, H, D), ref.reshape(B * N, H, D), torch.float16, "forced plan")


# 32-node workgroups (two 16-node groups per wave), forced where the default plan would pick
# 16: (B, H, S, D, N, kv_format, q dtype, lengths, splits)
NG2_CASES = [
    (1, 4, 700, 128, 17, "affine_block", torch.float16, [700], None),          # one node of the second group
    (2, 2, 257, 64, 40, "symmetric_token", torch.bfloat16, [257, 16], None),  # a workgroup with an empty group
    (2, 4, 1500, 128, 33, "affine_block", torch.bfloat16, [1500, 900], "3"),  # split partials, tail kernel
    (1, 2, 200, 64, 70, "affine_block", torch.float32, [200], "1"),           # fused tail, > 64 nodes
    (2, 4, 700, 128, 48, "affine_block", torch.bfloat16, [700, 333], "1"),    # fused tail, 1.5 workgroups
    (2, 4, 900, 128, 40, "fp8_block", torch.float16, [900, 512], None),       # FP8, two groups per wave
]


@pytest.mark.parametrize("B,H,S,D,N,fmt,q_dtype,lengths,splits", NG2_CASES)
def test_tree_mfma_32_node_workgroups(monkeypatch, B, H, S, D, N, fmt, q_dtype, lengths, splits):
    announce(f"tree mfma 32-node workgroups B{B} H{H} S{S} D{D} N{N} {fmt} {q_dtype} splits={splits}")
    monkeypatch.setenv("FLASHSPEC_TREE_NODES_PER_WG", "32")
    if splits is not None:
        monkeypatch.setenv("FLASHSPEC_NUM_SPLITS", splits)
    parents = _random_parents(B, N, S + 3 * N)
    got, ref, stats = _run(B, H, S, D, N, parents, lengths, kv_format=fmt, q_dtype=q_dtype, draft_dtype=q_dtype,
                           seed=S + 2 * N, kernel="mfma")
    assert stats["nodes_per_workgroup"] == 32.0
    if splits is not None:
        assert stats["num_splits"] == float(splits)
    assert_attention_close(got.reshape(B * N, H, D), ref.reshape(B * N, H, D), q_dtype, "32-node workgroups")


def test_tree_mfma_agrees_with_row_kernel():
    """Both prefix kernels on one input: within the attention tolerance of each other."""

    announce("tree mfma vs rows")
    B, H, S, D, N = 4, 8, 2048, 128, 16
    parents = _random_parents(B, N, 9)
    q = randn((B, N, H, D), 51).to(DEV)
    k, v = randn((B, H, S, D), 52).to(DEV), randn((B, H, S, D), 53).to(DEV)
    dk, dv = randn((B, N, H, D), 54).to(DEV), randn((B, N, H, D), 55).to(DEV)
    cache = fa.PagedKVCache.from_dense(k, v, 16, lengths=torch.tensor([2048, 1000, 17, 1600]).to(DEV),
                                       block_table_pattern="shuffled", layout_seed=4)
    par = torch.tensor(parents)
    a = fa.tree_verify_attention(q, cache, dk, dv, par, kernel="mfma")
    b = fa.tree_verify_attention(q, cache, dk, dv, par, kernel="rows")
    torch.cuda.synchronize(DEV)
    ref = ot.tree_verify_attention(np_of(q.cpu().float()), from_cache(cache), np_of(dk.cpu().float()),
                                   np_of(dv.cpu().float()), parents)
    assert_attention_close(a.reshape(B * N, H, D), ref.reshape(B * N, H, D), torch.float16, "mfma")
    assert_attention_close(b.reshape(B * N, H, D), ref.reshape(B * N, H, D), torch.float16, "rows")
    assert float((a.float() - b.float()).abs().max()) <= 2e-3


def test_tree_deep_chain_64_nodes():
    """A 64-node chain: the tail's register walk sets every bit of the path mask (node 63 sees
    all 64 drafts); with the prefix it is plain attention over prefix + chain."""

    announce("tree 64-node chain")
    B, H, S, D, N = 2, 2, 150, 128, 64
    parents = np.tile(np.arange(-1, N - 1), (B, 1))
    for kernel in ("mfma", "rows"):
        got, ref, _ = _run(B, H, S, D, N, parents, [150, 40], seed=61, kernel=kernel)
        assert_attention_close(got.reshape(B * N, H, D), ref.reshape(B * N, H, D), torch.float16, f"chain {kernel}")


@pytest.mark.parametrize("D,fmt,dtype,N", [(128, "affine_block", torch.float16, 16), (64, "symmetric_token", torch.bfloat16, 40),
                                          (256, "affine_block", torch.float32, 9), (128, "symmetric_token", torch.float16, 70),
                                          (128, "affine_block", torch.bfloat16, 48)])
def test_tree_mfma_fused_tail(monkeypatch, D, fmt, dtype, N):
    """One split and drafts in q's dtype: the multi-query kernel finishes the rows itself (its
    LDS-merged prefix state plus the path tokens; > 64 nodes walk parents in memory)."""

    announce(f"tree mfma fused tail D{D} {fmt} {dtype} N{N}")
    monkeypatch.setenv("FLASHSPEC_NUM_SPLITS", "1")
    B, H, S = 2, 4, 700
    parents = _random_parents(B, N, D + N)
    got, ref, stats = _run(B, H, S, D, N, parents, [700, 333], kv_format=fmt, q_dtype=dtype, draft_dtype=dtype,
                           seed=D + N, kernel="mfma")
    assert stats["num_splits"] == 1.0
    assert_attention_close(got.reshape(B * N, H, D), ref.reshape(B * N, H, D), dtype, "fused tail")


def test_tree_parents_cache_reuse_and_change():
    """A host parents tensor reused across calls is served from the device cache; changing its
    contents (in place) gives a different, correct tree."""

    announce("tree parents cache")
    B, H, S, D, N = 2, 4, 300, 128, 8
    q = randn((B, N, H, D), 71).to(DEV)
    k, v = randn((B, H, S, D), 72).to(DEV), randn((B, H, S, D), 73).to(DEV)
    dk, dv = randn((B, N, H, D), 74).to(DEV), randn((B, N, H, D), 75).to(DEV)
    cache = fa.PagedKVCache.from_dense(k, v, 16, block_table_pattern="shuffled", layout_seed=5)
    par = torch.tensor(_random_parents(B, N, 3))
    outs = []
    for _ in range(2):
        outs.append(fa.tree_verify_attention(q, cache, dk, dv, par))
    par.numpy()[0, 5] = -1  # in place, behind torch's version counter
    outs.append(fa.tree_verify_attention(q, cache, dk, dv, par))
    torch.cuda.synchronize(DEV)
    assert torch.equal(outs[0], outs[1])
    ref = ot.tree_verify_attention(np_of(q.cpu().float()), from_cache(cache), np_of(dk.cpu().float()),
                                   np_of(dv.cpu().float()), par.numpy())
    assert_attention_close(outs[2].reshape(B * N, H, D), ref.reshape(B * N, H, D), torch.float16, "changed tree")
    with pytest.raises(ValueError):
        bad = par.clone()
        bad[1, 2] = 5
        fa.tree_verify_attention(q, cache, dk, dv, bad)


@pytest.mark.parametrize("q_dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_tree_mfma_unaligned_queries(q_dtype):
    """Query rows that start one element past a 16-byte boundary are fetched value by value (and
    the drafts then walk global memory); both match the oracle, and each other to fp32 rounding."""

    announce(f"tree mfma unaligned queries {q_dtype}")
    B, H, S, D, N = 2, 8, 500, 128, 12
    parents = torch.tensor(_random_parents(B, N, 78)).to(DEV)
    q = randn((B, N, H, D), 96, torch.float32).to(q_dtype).to(DEV)
    k, v = randn((B, H, S, D), 97).to(DEV), randn((B, H, S, D), 98).to(DEV)
    dk = randn((B, N, H, D), 99, torch.float32).to(q_dtype).to(DEV)
    dv = randn((B, N, H, D), 100, torch.float32).to(q_dtype).to(DEV)
    cache = fa.PagedKVCache.from_dense(k, v, 16, lengths=torch.tensor([500, 233]).to(DEV))
    raw = torch.zeros(q.numel() + 1, dtype=q_dtype, device=DEV)
    q_off = raw[1:].view(B, N, H, D)
    q_off.copy_(q)
    assert q_off.data_ptr() % 16 != 0 and q_off.is_contiguous()
    a, st = fa.tree_verify_attention(q, cache, dk, dv, parents, return_stats=True, kernel="mfma")
    b = fa.tree_verify_attention(q_off, cache, dk, dv, parents, kernel="mfma")
    torch.cuda.synchronize(DEV)
    assert st["mfma_prefix"] == 1.0
    ref = ot.tree_verify_attention(np_of(q.float()), from_cache(cache), np_of(dk.float()), np_of(dv.float()),
                                   np_of(parents))
    assert_attention_close(a, ref, q_dtype, "aligned queries")
    assert_attention_close(b, ref, q_dtype, "unaligned queries")
    assert (a.float() - b.float()).abs().max().item() <= 2e-3


def test_tree_mfma_unaligned_drafts_walk_global_memory():
    """Draft tensors whose data does not start on a 16-byte boundary are not copied to LDS: each
    node's path is then walked in global memory, token by token, where aligned fp16 drafts enter
    the prefix states as MFMA tile pairs.  Both match the oracle, and each other to fp32 rounding."""

    announce("tree mfma unaligned drafts")
    B, H, S, D, N = 2, 8, 600, 128, 20
    parents = torch.tensor(_random_parents(B, N, 77)).to(DEV)
    q = randn((B, N, H, D), 91, torch.float32).to(torch.float16).to(DEV)
    k, v = randn((B, H, S, D), 92).to(DEV), randn((B, H, S, D), 93).to(DEV)
    dk = randn((B, N, H, D), 94, torch.float32).to(torch.float16).to(DEV)
    dv = randn((B, N, H, D), 95, torch.float32).to(torch.float16).to(DEV)
    cache = fa.PagedKVCache.from_dense(k, v, 16, lengths=torch.tensor([600, 311]).to(DEV))
    n = dk.numel()
    raw_k = torch.empty(n + 8, dtype=torch.float16, device=DEV)
    raw_v = torch.empty(n + 8, dtype=torch.float16, device=DEV)
    dk_off = raw_k[1:n + 1].view(B, N, H, D)  # 2 bytes past the allocation's start
    dv_off = raw_v[1:n + 1].view(B, N, H, D)
    dk_off.copy_(dk)
    dv_off.copy_(dv)
    assert dk_off.data_ptr() % 16 != 0 and dk_off.is_contiguous()
    a, st = fa.tree_verify_attention(q, cache, dk, dv, parents, return_stats=True, kernel="mfma")
    b = fa.tree_verify_attention(q, cache, dk_off, dv_off, parents, kernel="mfma")
    torch.cuda.synchronize(DEV)
    assert st["mfma_prefix"] == 1.0
    ref = ot.tree_verify_attention(np_of(q.float()), from_cache(cache), np_of(dk.float()), np_of(dv.float()),
                                   np_of(parents))
    assert_attention_close(a, ref, torch.float16, "aligned drafts")
    assert_attention_close(b, ref, torch.float16, "unaligned drafts")
    assert (a.float() - b.float()).abs().max().item() <= 2e-3
