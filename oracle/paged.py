"""Oracle: paged INT8 KV cache layout, append and allocator (test infrastructure only).

Restates reference src/flashspec/paged.py in numpy.  Physical pages are
``[P, heads, page, head_dim]`` quantized with quant block == page, so the
quantized arrays are ``values [P, H, 1, page, D]``, ``scale/zero [P, H, 1, 1, 1]``.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, List, Optional, Sequence

import numpy as np

from . import quant as oq

F32 = np.float32


@dataclass(frozen=True)
class OracleCache:
    """Mirror of ``PagedKVCache`` (paged.py:258-300)."""

    k_quant: oq.OracleQuant
    v_quant: oq.OracleQuant
    block_table: np.ndarray  # int64 [B, cols], -1 = unallocated
    lengths: np.ndarray  # int64 [B]
    block_size: int
    max_seq_len: int

    @property
    def batch_size(self) -> int:
        return int(self.block_table.shape[0])

    @property
    def num_heads(self) -> int:
        return int(self.k_quant.original_shape[1])

    @property
    def head_dim(self) -> int:
        return int(self.k_quant.original_shape[-1])


def interleaved_perm(batch: int, blocks_per_seq: int) -> np.ndarray:
    """``arange(B*n).reshape(B, n).T.flatten()`` — closed form of paged.py:392-393."""

    return np.arange(batch * blocks_per_seq, dtype=np.int64).reshape(batch, blocks_per_seq).T.reshape(-1)


def dense_to_pages(k: np.ndarray, block_size: int) -> np.ndarray:
    """[B, H, S, D] -> batch-major physical pages [B*n, H, page, D] (paged.py:343-370)."""

    B, H, S, D = k.shape
    n = (S + block_size - 1) // block_size
    padded = n * block_size
    if padded != S:
        k = np.concatenate([k, np.zeros((B, H, padded - S, D), dtype=k.dtype)], axis=2)
    return k.reshape(B, H, n, block_size, D).transpose(0, 2, 1, 3, 4).reshape(B * n, H, block_size, D)


def from_dense(
    k: np.ndarray,
    v: np.ndarray,
    block_size: int = 16,
    *,
    lengths: Optional[np.ndarray] = None,
    perm: Optional[np.ndarray] = None,
    kv_format: str = "affine_block",
) -> OracleCache:
    """``PagedKVCache.from_dense`` (paged.py:302-419) with an explicit physical permutation.

    ``perm[j]`` is the batch-major page stored at physical slot ``j``
    (``physical = pages[perm]``) and ``block_table = inverse(perm)``
    (paged.py:384-398).  ``perm=None`` is the contiguous layout.  ``kv_format="fp8_block"``
    quantizes the pages with the FP8 E4M3 per-page format of oracle/fp8.py, and
    ``"affine_channel"`` with per-page, per-channel affine INT8 (quant.quantize_int8_per_channel),
    instead of the reference's per-page affine INT8.
    """

    B, H, S, D = k.shape
    n = (S + block_size - 1) // block_size
    total = B * n
    pk = dense_to_pages(np.asarray(k, dtype=F32), block_size)
    pv = dense_to_pages(np.asarray(v, dtype=F32), block_size)
    table = np.arange(total, dtype=np.int64).reshape(B, n)
    if perm is not None:
        perm = np.asarray(perm, dtype=np.int64)
        pk, pv = pk[perm], pv[perm]
        inverse = np.empty_like(perm)
        inverse[perm] = np.arange(total, dtype=np.int64)
        table = inverse.reshape(B, n)
    if lengths is None:
        lens = np.full((B,), S, dtype=np.int64)
    else:
        lens = np.asarray(lengths, dtype=np.int64).copy()
        if lens.shape != (B,) or (lens < 0).any() or (lens > S).any():
            raise ValueError("lengths must be [batch] with values in [0, seq_len]")
    if kv_format == "affine_block":
        quantize = oq.quantize_int8_per_block
    elif kv_format == "affine_channel":
        quantize = oq.quantize_int8_per_channel
    elif kv_format == "fp8_block":
        from .fp8 import quantize_fp8_per_block as quantize
    else:
        raise ValueError("kv_format must be 'affine_block', 'affine_channel' or 'fp8_block'")
    return OracleCache(
        k_quant=quantize(pk, block_size),
        v_quant=quantize(pv, block_size),
        block_table=table,
        lengths=lens,
        block_size=block_size,
        max_seq_len=S,
    )


def to_dense(cache: OracleCache):
    """Dequantize the whole store, gather by ``table.clamp_min(0)``, crop (paged.py:421-461)."""

    pk = oq.dequantize(cache.k_quant)
    pv = oq.dequantize(cache.v_quant)
    table = np.maximum(cache.block_table, 0)
    B, H, D = cache.batch_size, cache.num_heads, cache.head_dim

    def gather(p):
        g = p[table]  # [B, cols, H, page, D]
        return g.transpose(0, 2, 1, 3, 4).reshape(B, H, -1, D)[:, :, : cache.max_seq_len, :]

    return gather(pk), gather(pv)


def append(cache: OracleCache, k_new: np.ndarray, v_new: np.ndarray) -> OracleCache:
    """``PagedKVCache.append`` (paged.py:463-557).

    Dequantizes the whole store, widens the table with -1 columns, gives each
    unallocated logical page a fresh zero page at the end of the store, writes
    the new rows, then requantizes the *whole* store with block == page.
    """

    B, H, T, D = k_new.shape
    bs = cache.block_size
    pk = oq.dequantize_int8_per_block(cache.k_quant).copy()
    pv = oq.dequantize_int8_per_block(cache.v_quant).copy()
    table = cache.block_table.copy()
    lengths = cache.lengths.copy()
    need = int(((lengths + T + bs - 1) // bs).max())
    if need > table.shape[1]:
        table = np.concatenate([table, np.full((B, need - table.shape[1]), -1, dtype=np.int64)], axis=1)
    kn = np.asarray(k_new, dtype=F32)
    vn = np.asarray(v_new, dtype=F32)
    for b in range(B):
        start = int(lengths[b])
        for t in range(T):
            pos = start + t
            lb, off = pos // bs, pos % bs
            phys = int(table[b, lb])
            if phys < 0:
                phys = pk.shape[0]
                zero = np.zeros((1, H, bs, D), dtype=F32)
                pk = np.concatenate([pk, zero])
                pv = np.concatenate([pv, zero])
                table[b, lb] = phys
            pk[phys, :, off, :] = kn[b, :, t, :]
            pv[phys, :, off, :] = vn[b, :, t, :]
    lengths = lengths + T
    return OracleCache(
        k_quant=oq.quantize_int8_per_block(pk, bs),
        v_quant=oq.quantize_int8_per_block(pv, bs),
        block_table=table,
        lengths=lengths,
        block_size=bs,
        max_seq_len=int(lengths.max()),
    )


class OracleAllocator:
    """``PagedKVAllocator`` page semantics (paged.py:17-255).

    Lowest-free-page allocation (``pop(0)``; the free list is re-sorted on
    release), prompt pages quantized from zero-filled blocks, and per-token
    append that dequantizes the touched page — stale rows of a reused page
    included — writes the row and requantizes only that page.
    """

    def __init__(self, capacity_blocks: int, heads: int, head_dim: int, block_size: int = 16):
        self.capacity_blocks, self.heads, self.head_dim, self.block_size = capacity_blocks, heads, head_dim, block_size
        zeros = np.zeros((capacity_blocks, heads, block_size, head_dim), dtype=F32)
        self.k_quant = oq.quantize_int8_per_block(zeros, block_size)
        self.v_quant = oq.quantize_int8_per_block(zeros, block_size)
        self.free: List[int] = list(range(capacity_blocks))
        self.requests: Dict[int, dict] = {}

    # -- page helpers (paged.py:221-255) ------------------------------------------------
    def _allocate(self) -> int:
        if not self.free:
            raise RuntimeError("allocator out of physical blocks")
        return self.free.pop(0)

    def _dequantized_block(self, idx: int):
        def one(q: oq.OracleQuant):
            sub = oq.OracleQuant(
                q.values[idx : idx + 1], q.scale[idx : idx + 1], q.zero_point[idx : idx + 1],
                self.block_size, (1, self.heads, self.block_size, self.head_dim),
            )
            return oq.dequantize_int8_per_block(sub).copy()

        return one(self.k_quant), one(self.v_quant)

    def _write_block(self, idx: int, kb: np.ndarray, vb: np.ndarray) -> None:
        for store, blk in ((self.k_quant, kb), (self.v_quant, vb)):
            q = oq.quantize_int8_per_block(blk, self.block_size)
            store.values[idx] = q.values[0]
            store.scale[idx] = q.scale[0]
            store.zero_point[idx] = q.zero_point[0]

    # -- lifecycle (paged.py:66-151) ------------------------------------------------------
    def add_request(self, rid: int, k: np.ndarray, v: np.ndarray, length: Optional[int] = None) -> None:
        if rid in self.requests:
            raise ValueError("request exists")
        S = k.shape[2]
        eff = S if length is None else int(length)
        need = (eff + self.block_size - 1) // self.block_size
        if len(self.free) < need:
            raise RuntimeError("allocator out of physical blocks")
        blocks = []
        for lb in range(need):
            idx = self._allocate()
            blocks.append(idx)
            start, end = lb * self.block_size, min((lb + 1) * self.block_size, eff)
            kb = np.zeros((1, self.heads, self.block_size, self.head_dim), dtype=F32)
            vb = np.zeros_like(kb)
            kb[:, :, : end - start] = np.asarray(k[:, :, start:end], dtype=F32)
            vb[:, :, : end - start] = np.asarray(v[:, :, start:end], dtype=F32)
            self._write_block(idx, kb, vb)
        self.requests[rid] = {"blocks": blocks, "length": eff}

    def append_request(self, rid: int, k_new: np.ndarray, v_new: np.ndarray) -> None:
        req = self.requests[rid]
        touched: Dict[int, tuple] = {}
        for t in range(k_new.shape[2]):
            pos = req["length"] + t
            lb, off = pos // self.block_size, pos % self.block_size
            if lb == len(req["blocks"]):
                req["blocks"].append(self._allocate())
            idx = req["blocks"][lb]
            if idx not in touched:
                touched[idx] = self._dequantized_block(idx)
            kb, vb = touched[idx]
            kb[:, :, off, :] = np.asarray(k_new[:, :, t, :], dtype=F32)
            vb[:, :, off, :] = np.asarray(v_new[:, :, t, :], dtype=F32)
        for idx, (kb, vb) in touched.items():
            self._write_block(idx, kb, vb)
        req["length"] += k_new.shape[2]

    def append_batch(self, rids: Sequence[int], k_new: np.ndarray, v_new: np.ndarray) -> None:
        for i, rid in enumerate(rids):
            self.append_request(rid, k_new[i : i + 1], v_new[i : i + 1])

    def release_request(self, rid: int) -> None:
        req = self.requests.pop(rid)
        self.free.extend(req["blocks"])
        self.free.sort()

    def to_cache(self, rids: Optional[Sequence[int]] = None) -> OracleCache:
        rids = list(self.requests) if rids is None else list(rids)
        reqs = [self.requests[r] for r in rids]
        cols = max(1, max(len(r["blocks"]) for r in reqs))
        table = np.full((len(reqs), cols), -1, dtype=np.int64)
        lengths = np.zeros((len(reqs),), dtype=np.int64)
        for i, r in enumerate(reqs):
            table[i, : len(r["blocks"])] = r["blocks"]
            lengths[i] = r["length"]
        return OracleCache(self.k_quant, self.v_quant, table, lengths, self.block_size, int(lengths.max()))
