"""Speculative-decoding tree verification over a paged INT8 prefix.

The reference plans this kernel (doc/TODO.MD:186-237) without implementing it.  Semantics:
request b carries N draft nodes in topological order with ``parents[b, n]`` in [-1, n)
(-1: the node hangs off the last committed token).  Node n attends to the committed prefix
(tokens [0, lengths[b]) of a ``PagedKVCache``) and to the draft tokens on its own root path
(n and its ancestors), never to siblings or other branches.  Draft K/V are unquantized.

On GPU, ``fs_tree_verify_i8`` runs a multi-query prefix kernel (one wave reads each prefix
tile once for 16 nodes, or 32 for larger trees where registers allow, with matrix-core products;
head_dim 64/128/256, pages of 16k tokens) or,
for other stores, the paged decode kernel with one query row per node; a tail merges the
prefix state with the path tokens (inside the prefix kernel when it runs one split).  On CPU
the dense tree-mask formulation runs in torch.
"""

from __future__ import annotations

import math
import os
from collections import OrderedDict
from typing import Any

import numpy as np
import torch

from . import _lib
from .paged import PagedKVCache
from .quant import build_compression_stats, is_fp8, is_per_channel
from .triton_utils import device_cu_count, launch_plan, merge_area, plan_tree_splits

__all__ = ["tree_verify_attention", "validate_parents", "path_mask", "tree_shape"]


def validate_parents(parents: torch.Tensor, batch: int, nodes: int) -> torch.Tensor:
    """Host copy of ``parents`` after checking it is a forest in topological order."""

    if parents.ndim != 2 or tuple(parents.shape) != (batch, nodes):
        raise ValueError(f"parents must be [batch, nodes] = [{batch}, {nodes}]")
    if parents.dtype not in (torch.int32, torch.int64):
        raise ValueError("parents must be an int32/int64 tensor")
    host = parents.detach().to("cpu", torch.int64).contiguous()
    a = host.numpy()
    if bool(((a < -1) | (a >= np.arange(nodes, dtype=np.int64))).any()):
        raise ValueError("parents[b, n] must lie in [-1, n): cycles, forward edges and orphans are invalid")
    return host


def path_mask(parents: torch.Tensor) -> torch.Tensor:
    """``mask[b, n, j]`` = draft node j lies on node n's root path (``parents`` validated)."""

    batch, nodes = parents.shape
    mask = torch.zeros((batch, nodes, nodes), dtype=torch.bool)
    for n in range(nodes):
        mask[:, n, n] = True
        par = parents[:, n]
        has = par >= 0
        if bool(has.any()):
            mask[has, n] |= mask[has, par[has]]
    return mask


def _validate(q, cache, draft_k, draft_v):
    if not isinstance(cache, PagedKVCache):
        raise ValueError("cache must be a PagedKVCache")
    if q.ndim != 4:
        raise ValueError("q must be [batch, nodes, heads, head_dim]")
    if draft_k.shape != q.shape or draft_v.shape != q.shape:
        raise ValueError("draft_k and draft_v must match q's [batch, nodes, heads, head_dim]")
    batch, nodes, heads, head_dim = (int(s) for s in q.shape)
    if batch != cache.batch_size or heads != cache.num_heads or head_dim != cache.head_dim:
        raise ValueError("q does not match the cache's batch, heads or head_dim")
    if nodes <= 0:
        raise ValueError("need at least one draft node")
    if head_dim > 256:
        raise ValueError("head_dim must be <= 256")
    kq, vq = cache.k_quant, cache.v_quant
    if is_fp8(kq) != is_fp8(vq) or is_per_channel(kq) != is_per_channel(vq):
        raise ValueError("k and v caches must share one KV format")
    return batch, nodes, heads, head_dim


def _portable(q, cache, draft_k, draft_v, parents_host):
    batch, nodes, heads, head_dim = q.shape
    kp, vp = cache.to_dense()  # [B, H, S, D] float32
    S = kp.shape[2]
    dev = kp.device
    keys = torch.cat([kp, draft_k.to(dev, torch.float32).permute(0, 2, 1, 3)], dim=2)
    vals = torch.cat([vp, draft_v.to(dev, torch.float32).permute(0, 2, 1, 3)], dim=2)
    allowed = torch.zeros((batch, nodes, S + nodes), dtype=torch.bool, device=dev)
    allowed[:, :, :S] = torch.arange(S, device=dev)[None, None, :] < cache.lengths.to(dev)[:, None, None]
    allowed[:, :, S:] = path_mask(parents_host).to(dev)
    scores = torch.einsum("bnhd,bhkd->bhnk", q.to(dev, torch.float32), keys) / math.sqrt(head_dim)
    scores = scores.masked_fill(~allowed[:, None], torch.finfo(torch.float32).min)
    out = torch.einsum("bhnk,bhkd->bnhd", torch.softmax(scores, dim=-1), vals)
    return out.to(q.dtype)


_KERNELS = {"auto": 0, "rows": 1, "mfma": 2}


def _hip(q, cache, draft_k, draft_v, parents_dev, dims, kernel):
    batch, nodes, heads, head_dim = dims
    lib = _lib.require()
    dev = q.device
    kq, vq = cache.k_quant, cache.v_quant
    if draft_k.device != dev or draft_v.device != dev or cache.block_table.device != dev:
        raise RuntimeError("q, draft K/V and the cache must be on the same GPU")
    if q.dtype not in _lib.DTYPE_CODE or draft_k.dtype not in _lib.DTYPE_CODE or draft_v.dtype != draft_k.dtype:
        raise ValueError("q and draft K/V must be float32, float16 or bfloat16 (draft_k and draft_v alike)")
    q_c, dk_c, dv_c = q.contiguous(), draft_k.contiguous(), draft_v.contiguous()
    table = cache.block_table.contiguous()
    lengths = cache.lengths.to(torch.int64).contiguous()
    rows = batch * nodes * heads
    max_seq_len = int(cache.max_seq_len)
    fp8, per_channel = is_fp8(kq), is_per_channel(kq)
    mfma_ok = not per_channel and bool(lib.fs_tree_mfma_path(head_dim, int(cache.block_size), int(kq.block_size)))
    if kernel == "mfma" and not mfma_ok:
        raise ValueError("kernel='mfma' needs per-block or per-token parameters (INT8 or FP8), head_dim 64/128/256, "
                         "pages of a multiple of 16 tokens and quant blocks of 1 or a multiple of 16 tokens")
    use_mfma = mfma_ok and kernel != "rows"
    if use_mfma:
        cu = device_cu_count(dev)
        qcode, qb = _lib.dtype_code(q.dtype), int(kq.block_size)
        per_wg = int(lib.fs_tree_nodes_per_workgroup(head_dim, nodes, qcode, qb, batch * heads, cu))
        forced = os.environ.get("FLASHSPEC_TREE_NODES_PER_WG")
        if forced == "16" or (forced == "32" and nodes > 16 and
                              lib.fs_tree_nodes_per_workgroup(head_dim, nodes, qcode, qb, batch * heads, 0) == 32):
            per_wg = int(forced)  # 32 only where a wave has the registers for it
        units = batch * heads * math.ceil(nodes / per_wg)
        split_tiles, max_splits, waves = plan_tree_splits(max_seq_len, units, head_dim, cu)
        tiled, block_n = True, 16
    else:
        tiled, waves, split_tiles, max_splits, block_n = launch_plan(max_seq_len, rows, head_dim,
                                                                     int(cache.block_size), int(kq.block_size), dev,
                                                                     per_channel=per_channel)
    out = torch.empty_like(q_c)
    stream = _lib.stream_ptr(dev)
    plan = {"num_splits": float(max_splits), "split_tiles": float(split_tiles), "num_warps": float(waves),
            "block_n": float(block_n), "tiled_path": float(tiled), "mfma_prefix": float(use_mfma),
            "nodes_per_workgroup": float(per_wg if use_mfma else 1)}
    if use_mfma and dk_c.dtype == q_c.dtype:
        # the multi-query kernel finishes every row itself: split rows merge inside the launch
        area, area_bytes = merge_area(dev, rows, max_splits, head_dim, stream) if max_splits > 1 else (None, 0)
        _lib.check(lib.fs_tree_verify_merged(
            q_c.data_ptr(), _lib.dtype_code(q_c.dtype), 1 if fp8 else 0, kq.values.data_ptr(), kq.scale.data_ptr(),
            None if fp8 else kq.zero_point.data_ptr(), vq.values.data_ptr(), vq.scale.data_ptr(),
            None if fp8 else vq.zero_point.data_ptr(), table.data_ptr(), table.element_size(), int(table.shape[1]),
            lengths.data_ptr(), dk_c.data_ptr(), dv_c.data_ptr(), parents_dev.data_ptr(), out.data_ptr(),
            _lib.ptr(area), area_bytes, batch, nodes, heads, head_dim, int(kq.values.shape[0]),
            int(cache.block_size), int(kq.block_size), max_seq_len, 1.0 / math.sqrt(head_dim), split_tiles,
            max_splits, waves, per_wg, stream))
        return out, plan
    ws_bytes = int(lib.fs_decode_workspace_bytes(rows, max_splits, head_dim))
    workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    store = ([kq.values.data_ptr(), kq.scale.data_ptr(), vq.values.data_ptr(), vq.scale.data_ptr()] if fp8 else
             [kq.values.data_ptr(), kq.scale.data_ptr(), kq.zero_point.data_ptr(), vq.values.data_ptr(),
              vq.scale.data_ptr(), vq.zero_point.data_ptr()])
    entry = lib.fs_tree_verify_fp8 if fp8 else (lib.fs_tree_verify_i8_channel if per_channel else lib.fs_tree_verify_i8)
    _lib.check(entry(
        q_c.data_ptr(), _lib.dtype_code(q_c.dtype), *store,
        table.data_ptr(), table.element_size(), int(table.shape[1]), lengths.data_ptr(), dk_c.data_ptr(),
        dv_c.data_ptr(), _lib.dtype_code(dk_c.dtype), parents_dev.data_ptr(), out.data_ptr(), workspace.data_ptr(),
        ws_bytes, batch, nodes, heads, head_dim, int(kq.values.shape[0]), int(cache.block_size), int(kq.block_size),
        max_seq_len, 1.0 / math.sqrt(head_dim), split_tiles, max_splits, waves,
        (3 if per_wg == 16 else 4) if use_mfma else 1, stream))
    return out, plan


def tree_verify_attention(q: torch.Tensor, cache: PagedKVCache, draft_k: torch.Tensor, draft_v: torch.Tensor,
                          parents: torch.Tensor, return_stats: bool = False, validate: bool = True,
                          kernel: str = "auto") -> Any:
    """Attention of every draft node over the prefix and its root path.

    ``q``, ``draft_k``, ``draft_v``: ``[batch, nodes, heads, head_dim]``; ``parents``:
    ``[batch, nodes]`` int with ``parents[b, n]`` in [-1, n).  Returns ``[batch, nodes, heads,
    head_dim]`` in q's dtype (and a stats dict with ``return_stats``).  ``ValueError`` for a
    malformed tree or shapes, ``RuntimeError`` for device mismatches or a GPU tensor without
    the HIP library.

    ``parents`` on the CPU (the usual case: the drafter builds the tree on the host) is
    checked there and copied to the GPU through pinned memory without waiting for the
    device; the validated device copy is kept (by content) for later calls with the same
    topology.  ``parents`` already on the GPU is copied back to check it, which waits for
    the device; ``validate=False`` skips that check, and the kernel then ends a node's path
    at the first parent outside [-1, own index) (never reading out of bounds).

    ``kernel`` picks the GPU prefix kernel: ``"mfma"`` reads each prefix tile once for 16
    (or 32) nodes with matrix-core products (head_dim 64/128/256, pages of 16k tokens, quant blocks
    of 1 or 16k tokens), ``"rows"`` runs the paged decode with one query row per node (any
    store), ``"auto"`` the first where it applies.
    """

    if kernel not in _KERNELS:
        raise ValueError(f"kernel must be one of {sorted(_KERNELS)}")
    dims = _validate(q, cache, draft_k, draft_v)
    batch, nodes, heads, head_dim = dims
    parents_host = None
    if q.device.type == "cuda":
        if parents.device.type == "cpu":
            parents_dev = _device_parents(parents, batch, nodes, q.device)
            parents_host = parents
        elif validate:
            parents_host = validate_parents(parents, batch, nodes)
            parents_dev = parents.to(torch.int64).contiguous()
        else:
            if parents.ndim != 2 or tuple(parents.shape) != (batch, nodes) or \
                    parents.dtype not in (torch.int32, torch.int64):
                raise ValueError(f"parents must be an int32/int64 [batch, nodes] = [{batch}, {nodes}] tensor")
            parents_dev = parents.to(torch.int64).contiguous()
        out, plan = _hip(q, cache, draft_k, draft_v, parents_dev, dims, kernel)
        materializes = False
    else:
        parents_host = validate_parents(parents, batch, nodes)
        out, plan = _portable(q, cache, draft_k, draft_v, parents_host), {}
        materializes = True
    if not return_stats:
        return out
    dense_bytes = 2 * batch * heads * int(cache.max_seq_len) * head_dim * q.element_size()
    shape = tree_shape(parents_host) if parents_host is not None else {}
    stats = build_compression_stats(dense_bytes, cache.estimated_bytes(), materializes_dense_kv=materializes,
                                    tree_nodes=float(nodes), tree_depth=float(shape.get("depth", float("nan"))),
                                    tree_leaves=float(shape.get("leaves", float("nan"))),
                                    tree_max_branch=float(shape.get("max_branch", float("nan"))), **plan)
    return out, stats


# Validated device copies of host parents tensors, keyed by content: a drafter with a static
# tree topology (one parents tensor reused every step) pays neither the check nor the copy
# after the first call.  A copy made on another stream is waited for through its event.
_PARENTS_CACHE: "OrderedDict[tuple, tuple]" = OrderedDict()
_PARENTS_CACHE_ENTRIES = 16


def _device_parents(parents: torch.Tensor, batch: int, nodes: int, dev: torch.device) -> torch.Tensor:
    host = parents.detach().to(torch.int64).contiguous()
    if tuple(host.shape) != (batch, nodes):
        raise ValueError(f"parents must be [batch, nodes] = [{batch}, {nodes}]")
    key = (dev.index, batch, nodes, host.numpy().tobytes())
    stream = torch.cuda.current_stream(dev)
    hit = _PARENTS_CACHE.get(key)
    if hit is not None:
        _PARENTS_CACHE.move_to_end(key)
        return _reuse_on(hit, stream)
    validate_parents(parents, batch, nodes)
    tensor = host.pin_memory().to(dev, non_blocking=True)
    ready = torch.cuda.Event()
    ready.record(stream)
    _PARENTS_CACHE[key] = (tensor, stream, ready)
    if len(_PARENTS_CACHE) > _PARENTS_CACHE_ENTRIES:
        _PARENTS_CACHE.popitem(last=False)
    return tensor


def _reuse_on(entry: tuple, stream) -> torch.Tensor:
    """A cached device copy ``(tensor, made_on, ready)`` used on ``stream``.

    On another stream than the one that made it, the stream first waits for the copy, and
    ``record_stream`` tells the caching allocator that ``stream`` uses the memory: once the
    entry is evicted, the block is then not handed out again until the kernels queued on
    ``stream`` up to that point have finished reading it.
    """

    tensor, made_on, ready = entry
    if made_on != stream:
        stream.wait_event(ready)
        tensor.record_stream(stream)
    return tensor


def tree_shape(parents: torch.Tensor) -> dict:
    """Largest depth (nodes on a root path), leaf count and branching factor over the batch of
    a validated ``parents`` (host or device tensor; [batch, nodes])."""

    a = parents.detach().to("cpu", torch.int64).numpy()
    batch, nodes = a.shape
    if nodes == 0:
        return {"depth": 0, "leaves": 0, "max_branch": 0}
    depth = np.ones((batch, nodes), dtype=np.int64)
    for n in range(nodes):
        par = a[:, n]
        has = par >= 0
        depth[has, n] = depth[has, par[has]] + 1
    children = np.zeros((batch, nodes + 1), dtype=np.int64)  # column nodes: children of the root
    for b in range(batch):
        np.add.at(children[b], np.where(a[b] >= 0, a[b], nodes), 1)
    leaves = int((children[:, :nodes] == 0).sum(axis=1).max())
    return {"depth": int(depth.max()), "leaves": leaves, "max_branch": int(children.max())}
