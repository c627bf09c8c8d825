"""Paged INT8 KV cache and allocator (reference src/flashspec/paged.py).

Physical page store: ``[num_pages, heads, page, head_dim]`` quantized with
quant block == page, i.e. ``values [P, H, 1, page, D]`` and ``scale/zero
[P, H, 1, 1, 1]``.  ``block_table [batch, cols]`` (int64, -1 = unallocated)
maps logical pages to physical ones.

On GPU every quantized write goes through the HIP page kernels:
``fs_quantize_pages_i8`` for ``from_dense`` and ``fs_update_pages_i8`` for
``append`` (whole-store requantization, as the reference does) and for the
allocator's prompt/append writes (only the touched pages).  Host bookkeeping —
free list, tables, lengths — stays in Python like the reference's.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, Sequence, Tuple

import numpy as np
import torch

from . import _lib
from .quant import (FP8_DTYPE, QuantizedTensor, dequantize_int8_per_block, estimate_quantized_bytes, is_fp8,
                    is_per_channel, quantize_fp8_per_block, quantize_int8_per_block, quantize_int8_per_channel,
                    quantize_int8_symmetric_per_token)

_SCALE_FLOOR = 1.0e-8  # quantizing an all-zero block gives int8 -128, scale fp32(1e-8), zero 0


def _normalize_device(device: torch.device | str) -> torch.device:
    dev = torch.device(device)
    if dev.type == "cuda" and dev.index is None:
        dev = torch.device("cuda", torch.cuda.current_device())
    return dev


def _empty_page_store(pages: int, heads: int, page: int, dim: int, device: torch.device, per_channel: bool = False):
    values = torch.empty((pages, heads, 1, page, dim), dtype=torch.int8, device=device)
    params = dim if per_channel else 1
    scale = torch.empty((pages, heads, 1, 1, params), dtype=torch.float32, device=device)
    zero = torch.empty((pages, heads, 1, 1, params), dtype=torch.int16, device=device)
    return values, scale, zero


def _src_for_kernel(x: torch.Tensor) -> torch.Tensor:
    if x.dtype not in _lib.DTYPE_CODE:
        x = x.to(torch.float32)
    return x.contiguous()


def _update_pages(store: QuantizedTensor, out: Tuple[torch.Tensor, torch.Tensor, torch.Tensor] | None,
                  pages: np.ndarray | None, n_pages: int, fresh: np.ndarray | None, row_src: np.ndarray,
                  src: torch.Tensor, *, heads: int, page: int, dim: int) -> None:
    """One ``fs_update_pages_i8`` call; ``out=None`` updates ``store`` in place."""

    lib = _lib.require()
    dev = store.values.device
    in_values = store.values.contiguous()
    in_scale = store.scale.contiguous()
    in_zero = store.zero_point.contiguous()
    in_pages = int(store.original_shape[0])
    in_qb = int(store.block_size)
    if out is None:
        if not (store.values.is_contiguous() and store.scale.is_contiguous() and store.zero_point.is_contiguous()):
            raise ValueError("in-place page update needs a contiguous store")
        out_values, out_scale, out_zero = in_values, in_scale, in_zero
    else:
        out_values, out_scale, out_zero = out
    src_t = _src_for_kernel(src)
    rs = torch.from_numpy(np.ascontiguousarray(row_src, dtype=np.int32)).to(dev, non_blocking=False)
    pg = None if pages is None else torch.from_numpy(np.ascontiguousarray(pages, dtype=np.int64)).to(dev)
    fr = None if fresh is None else torch.from_numpy(np.ascontiguousarray(fresh, dtype=np.uint8)).to(dev)
    _lib.check(lib.fs_update_pages_i8(
        in_values.data_ptr(), in_scale.data_ptr(), in_zero.data_ptr(), in_pages, in_qb,
        out_values.data_ptr(), out_scale.data_ptr(), out_zero.data_ptr(),
        _lib.ptr(pg), _lib.ptr(fr), n_pages, rs.data_ptr(), src_t.data_ptr(), _lib.dtype_code(src_t.dtype),
        int(src_t.shape[2]), heads, page, dim, _lib.stream_ptr(dev)))
    # rs/pg/fr/src_t may be freed now: the caching allocator hands their blocks out again
    # only to work ordered after this launch on the same stream.


@dataclass
class _RequestBlocks:
    logical_blocks: list[int]
    length: int


class PagedKVAllocator:
    """Fixed-capacity page allocator for the serving simulation (paged.py:17-255).

    Lowest-free-page allocation, per-request logical page lists, page reuse after
    release, and per-page requantization on append.
    """

    def __init__(self, *, capacity_blocks: int, heads: int, head_dim: int, block_size: int = 16,
                 device: torch.device | str = "cpu", dtype: torch.dtype = torch.float32) -> None:
        if capacity_blocks <= 0:
            raise ValueError("capacity_blocks must be positive")
        if heads <= 0 or head_dim <= 0:
            raise ValueError("heads and head_dim must be positive")
        if block_size <= 0:
            raise ValueError("block_size must be positive")
        self.capacity_blocks = int(capacity_blocks)
        self.heads = int(heads)
        self.head_dim = int(head_dim)
        self.block_size = int(block_size)
        self.device = _normalize_device(device)
        self.dtype = dtype
        shape = (self.capacity_blocks, self.heads, self.block_size, self.head_dim)
        if self.device.type == "cuda":
            # An all-zero page quantizes to int8 -128 with scale fp32(1e-8) and zero 0.
            self.k_quant = self._zero_store(shape)
            self.v_quant = self._zero_store(shape)
        else:
            empty = torch.zeros(shape, device=self.device, dtype=torch.float32)
            self.k_quant = quantize_int8_per_block(empty, block_size=self.block_size)
            self.v_quant = quantize_int8_per_block(empty, block_size=self.block_size)
        self._free_blocks = list(range(self.capacity_blocks))
        self._requests: dict[int, _RequestBlocks] = {}

    def _zero_store(self, shape) -> QuantizedTensor:
        values, scale, zero = _empty_page_store(shape[0], shape[1], shape[2], shape[3], self.device)
        values.fill_(-128)
        scale.fill_(_SCALE_FLOOR)
        zero.zero_()
        return QuantizedTensor(values, scale, zero, self.block_size, tuple(shape))

    @property
    def live_request_ids(self) -> list[int]:
        return list(self._requests.keys())

    # -- lifecycle ------------------------------------------------------------------------
    def add_request(self, request_id: int, k: torch.Tensor, v: torch.Tensor, *, length: int | None = None) -> None:
        """Allocate and write the prompt pages of one request (paged.py:66-106)."""

        request_id = int(request_id)
        if request_id in self._requests:
            raise ValueError(f"request_id {request_id} already exists")
        self._validate_kv(k, v, batch_expected=None)
        if k.shape[0] != 1:
            raise ValueError("add_request takes the KV of a single request (batch dim 1)")
        seq_len = int(k.shape[2])
        effective_length = seq_len if length is None else int(length)
        if effective_length < 0 or effective_length > seq_len:
            raise ValueError("length must be in [0, seq_len]")
        blocks_needed = (effective_length + self.block_size - 1) // self.block_size
        if len(self._free_blocks) < blocks_needed:
            raise RuntimeError("PagedKVAllocator is out of physical blocks")
        logical_blocks = [self._allocate_block() for _ in range(blocks_needed)]
        if blocks_needed:
            if self.device.type == "cuda":
                row_src = np.full((blocks_needed, self.block_size), -1, dtype=np.int32)
                for lb in range(blocks_needed):
                    start = lb * self.block_size
                    width = max(0, min(self.block_size, effective_length - start))
                    row_src[lb, :width] = np.arange(start, start + width)
                pages = np.asarray(logical_blocks, dtype=np.int64)
                fresh = np.ones(blocks_needed, dtype=np.uint8)
                for store, src in ((self.k_quant, k), (self.v_quant, v)):
                    _update_pages(store, None, pages, blocks_needed, fresh, row_src, src,
                                  heads=self.heads, page=self.block_size, dim=self.head_dim)
            else:
                for lb, physical_idx in enumerate(logical_blocks):
                    start = lb * self.block_size
                    end = min(start + self.block_size, effective_length)
                    kb = torch.zeros((1, self.heads, self.block_size, self.head_dim), device=self.device)
                    vb = torch.zeros_like(kb)
                    kb[:, :, : end - start] = k[:, :, start:end].to(device=self.device, dtype=torch.float32)
                    vb[:, :, : end - start] = v[:, :, start:end].to(device=self.device, dtype=torch.float32)
                    self._write_quantized_block(physical_idx, kb, vb)
        self._requests[request_id] = _RequestBlocks(logical_blocks=logical_blocks, length=effective_length)

    def _plan_append(self, request: _RequestBlocks, tokens: int, touched: Dict[int, list]) -> None:
        """Allocate pages crossed by `tokens` new rows; record (offset, token) per touched page."""

        for token_idx in range(tokens):
            position = request.length + token_idx
            logical_block, offset = divmod(position, self.block_size)
            if logical_block == len(request.logical_blocks):
                request.logical_blocks.append(self._allocate_block())
            touched.setdefault(request.logical_blocks[logical_block], []).append((offset, token_idx))

    def append_request(self, request_id: int, k_new: torch.Tensor, v_new: torch.Tensor) -> None:
        """Append tokens to one request; requantize only the touched pages (paged.py:108-136).

        A touched page is dequantized whole — stale rows of a reused page included —
        before the new rows are written, exactly as the reference does.
        """

        self._validate_kv(k_new, v_new, batch_expected=1)
        request = self._get_request(request_id)
        tokens = int(k_new.shape[2])
        if tokens <= 0:
            raise ValueError("appended token dimension must be non-empty")
        if self.device.type == "cuda":
            touched: Dict[int, list] = {}
            self._plan_append(request, tokens, touched)
            self._write_touched([(touched, 0)], tokens, k_new, v_new)
        else:
            touched_cpu: dict[int, tuple[torch.Tensor, torch.Tensor]] = {}
            k32 = k_new.to(device=self.device, dtype=torch.float32)
            v32 = v_new.to(device=self.device, dtype=torch.float32)
            for token_idx in range(tokens):
                position = request.length + token_idx
                logical_block, offset = divmod(position, self.block_size)
                if logical_block == len(request.logical_blocks):
                    request.logical_blocks.append(self._allocate_block())
                physical_idx = request.logical_blocks[logical_block]
                if physical_idx not in touched_cpu:
                    touched_cpu[physical_idx] = self._dequantized_block(physical_idx)
                kb, vb = touched_cpu[physical_idx]
                kb[:, :, offset, :] = k32[:, :, token_idx, :]
                vb[:, :, offset, :] = v32[:, :, token_idx, :]
            for physical_idx, (kb, vb) in touched_cpu.items():
                self._write_quantized_block(physical_idx, kb, vb)
        request.length += tokens

    def _write_touched(self, plans: list, tokens: int, k_src: torch.Tensor, v_src: torch.Tensor) -> None:
        """One page-update launch per tensor for every (touched-pages, source-entry) plan."""

        pages, rows = [], []
        for touched, entry in plans:
            for physical_idx, writes in touched.items():
                row = np.full(self.block_size, -1, dtype=np.int32)
                for offset, token_idx in writes:
                    row[offset] = entry * tokens + token_idx
                pages.append(physical_idx)
                rows.append(row)
        if not pages:
            return
        page_arr = np.asarray(pages, dtype=np.int64)
        row_src = np.stack(rows)
        for store, src in ((self.k_quant, k_src), (self.v_quant, v_src)):
            _update_pages(store, None, page_arr, len(pages), None, row_src, src,
                          heads=self.heads, page=self.block_size, dim=self.head_dim)

    def append_batch(self, request_ids: Sequence[int], k_new: torch.Tensor, v_new: torch.Tensor) -> None:
        """Append one slice of ``k_new/v_new`` per request, in order (paged.py:138-144).

        On GPU all requests' touched pages are rewritten by one launch per tensor;
        distinct requests never share a page.
        """

        request_ids = [int(r) for r in request_ids]
        self._validate_kv(k_new, v_new, batch_expected=len(request_ids))
        if self.device.type != "cuda" or len(set(request_ids)) != len(request_ids):
            for batch_idx, request_id in enumerate(request_ids):
                self.append_request(request_id, k_new[batch_idx: batch_idx + 1], v_new[batch_idx: batch_idx + 1])
            return
        tokens = int(k_new.shape[2])
        requests = [self._get_request(r) for r in request_ids]
        plans = []
        for entry, request in enumerate(requests):
            touched: Dict[int, list] = {}
            self._plan_append(request, tokens, touched)
            plans.append((touched, entry))
        self._write_touched(plans, tokens, k_new, v_new)
        for request in requests:
            request.length += tokens

    def shuffle_free_blocks(self, seed: int) -> None:
        """Put the free list in a seeded random order, so later allocations scatter over the pool.

        Not in the reference allocator, whose free list stays sorted (lowest page first);
        ``release_request`` restores that sorted order.
        """

        g = torch.Generator()
        g.manual_seed(int(seed))
        order = torch.randperm(len(self._free_blocks), generator=g).tolist()
        self._free_blocks = [self._free_blocks[i] for i in order]

    def release_request(self, request_id: int) -> None:
        """Return a request's pages to the free list (kept sorted; paged.py:146-151)."""

        request = self._requests.pop(int(request_id))
        self._free_blocks.extend(request.logical_blocks)
        self._free_blocks.sort()

    def to_cache(self, request_ids: Sequence[int] | None = None) -> "PagedKVCache":
        """Export live requests as a PagedKVCache, table padded with -1 (paged.py:153-179)."""

        ordered = self.live_request_ids if request_ids is None else [int(r) for r in request_ids]
        if not ordered:
            raise ValueError("to_cache needs at least one live request")
        requests = [self._get_request(r) for r in ordered]
        max_blocks = max(1, max((len(r.logical_blocks) for r in requests), default=0))
        table = torch.full((len(requests), max_blocks), -1, dtype=torch.int64)
        lengths = torch.empty((len(requests),), dtype=torch.int64)
        for i, r in enumerate(requests):
            if r.logical_blocks:
                table[i, : len(r.logical_blocks)] = torch.tensor(r.logical_blocks, dtype=torch.int64)
            lengths[i] = r.length
        return PagedKVCache(
            k_quant=self.k_quant,
            v_quant=self.v_quant,
            block_table=table.to(self.device),
            lengths=lengths.to(self.device),
            block_size=self.block_size,
            max_seq_len=int(lengths.max().item()),
        )

    def stats(self) -> Dict[str, float]:
        """Utilization and fragmentation (paged.py:181-199)."""

        allocated_blocks = self.capacity_blocks - len(self._free_blocks)
        used_tokens = sum(r.length for r in self._requests.values())
        allocated_tokens = allocated_blocks * self.block_size
        capacity_tokens = self.capacity_blocks * self.block_size
        padding_waste = max(0, allocated_tokens - used_tokens)
        return {
            "allocated_blocks": float(allocated_blocks),
            "free_blocks": float(len(self._free_blocks)),
            "live_requests": float(len(self._requests)),
            "used_tokens": float(used_tokens),
            "capacity_tokens": float(capacity_tokens),
            "block_utilization": used_tokens / max(1, allocated_tokens),
            "capacity_utilization": used_tokens / max(1, capacity_tokens),
            "padding_waste": float(padding_waste),
            "fragmentation": padding_waste / max(1, allocated_tokens),
        }

    # -- helpers ------------------------------------------------------------------------------
    def _validate_kv(self, k: torch.Tensor, v: torch.Tensor, *, batch_expected: int | None) -> None:
        """New tokens must be a pair of equal [batch, heads, tokens >= 1, head_dim] tensors on the pool's
        device; every violation is a ValueError, as for the reference allocator (paged.py:201-213)."""

        if (k.ndim, v.ndim) != (4, 4):
            raise ValueError(f"new K/V must be 4-D [batch, heads, tokens, head_dim] (got {k.ndim}-D / {v.ndim}-D)")
        if k.shape != v.shape:
            raise ValueError(f"new K and V differ in shape: {tuple(k.shape)} vs {tuple(v.shape)}")
        expect = {0: batch_expected, 1: self.heads, 3: self.head_dim}
        off = [f"dim {d} is {k.shape[d]}, expected {want}" for d, want in expect.items()
               if want is not None and k.shape[d] != want]
        if off:
            raise ValueError("new K/V do not fit this pool (batch = requests, heads, head_dim): " + "; ".join(off))
        if k.shape[2] < 1:
            raise ValueError("new K/V hold no tokens")
        if not (k.device == v.device == self.device):
            raise ValueError(f"new K/V must live on {self.device} (got {k.device} / {v.device})")

    def _get_request(self, request_id: int) -> _RequestBlocks:
        request = self._requests.get(int(request_id))
        if request is None:
            raise KeyError(f"no live request with id {request_id}")
        return request

    def _allocate_block(self) -> int:
        if not self._free_blocks:
            raise RuntimeError("PagedKVAllocator is out of physical blocks")
        return self._free_blocks.pop(0)

    def _dequantized_block(self, physical_idx: int) -> tuple[torch.Tensor, torch.Tensor]:
        shape = (1, self.heads, self.block_size, self.head_dim)

        def one(q: QuantizedTensor) -> torch.Tensor:
            sub = QuantizedTensor(q.values[physical_idx: physical_idx + 1], q.scale[physical_idx: physical_idx + 1],
                                  q.zero_point[physical_idx: physical_idx + 1], self.block_size, shape)
            return dequantize_int8_per_block(sub, dtype=torch.float32).clone()

        return one(self.k_quant), one(self.v_quant)

    def _write_quantized_block(self, physical_idx: int, k_block: torch.Tensor, v_block: torch.Tensor) -> None:
        for store, block in ((self.k_quant, k_block), (self.v_quant, v_block)):
            q = quantize_int8_per_block(block, block_size=self.block_size)
            store.values[physical_idx] = q.values[0]
            store.scale[physical_idx] = q.scale[0]
            store.zero_point[physical_idx] = q.zero_point[0]


def _layout_permutation(pattern: str, batch: int, blocks_per_seq: int, layout_seed: int,
                        device: torch.device) -> torch.Tensor | None:
    """Physical slot -> batch-major logical page (paged.py:376-398); None = contiguous."""

    total = batch * blocks_per_seq
    if pattern in {"shuffled", "random"}:
        generator = torch.Generator(device=device)
        generator.manual_seed(int(layout_seed))
        return torch.randperm(total, generator=generator, device=device)
    if pattern == "interleaved":
        return torch.arange(total, dtype=torch.int64, device=device).reshape(batch, blocks_per_seq).t().reshape(-1)
    return None


@dataclass(frozen=True)
class PagedKVCache:
    """Paged INT8 KV cache (paged.py:258-300).

    ``k_quant/v_quant`` hold the physical store (``original_shape = [P, H, page, D]``),
    ``block_table [batch, cols]`` maps logical to physical pages (-1 = unallocated),
    ``lengths [batch]`` the valid tokens per row, ``max_seq_len`` the attention span.
    """

    k_quant: QuantizedTensor
    v_quant: QuantizedTensor
    block_table: torch.Tensor
    lengths: torch.Tensor
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

    @classmethod
    def from_dense(cls, k: torch.Tensor, v: torch.Tensor, block_size: int = 16, *,
                   lengths: torch.Tensor | None = None, block_table_pattern: str = "contiguous",
                   layout_seed: int = 0, kv_format: str = "affine_block") -> "PagedKVCache":
        """Build a paged cache from dense ``[batch, heads, seq, dim]`` K/V (paged.py:302-419).

        Layouts: ``contiguous`` (batch-major), ``shuffled``/``random`` (seeded
        ``torch.randperm`` on k's device) and ``interleaved`` (logical-page-major).
        Only the physical placement changes; the logical K/V is identical.

        ``kv_format`` (not in the reference): ``affine_block`` quantizes each page per head
        as the reference does; ``symmetric_token`` stores symmetric absmax INT8 with one scale
        per token (``quantize_int8_symmetric_per_token``, quant block 1); ``fp8_block`` stores
        FP8 E4M3 codes with one scale per page and head (``quantize_fp8_per_block``);
        ``affine_channel`` stores affine INT8 with one scale / zero point per page, head and
        channel (``quantize_int8_per_channel``).
        """

        if kv_format not in ("affine_block", "symmetric_token", "fp8_block", "affine_channel"):
            raise ValueError("kv_format must be affine_block, symmetric_token, fp8_block or affine_channel")

        if k.ndim != 4 or v.ndim != 4:
            raise ValueError("k and v must be [batch, heads, seq_len, head_dim]")
        if k.shape != v.shape:
            raise ValueError("k and v must have the same shape")
        if block_size <= 0:
            raise ValueError("block_size must be positive")
        pattern = block_table_pattern.strip().lower()
        if pattern not in {"contiguous", "", "shuffled", "random", "interleaved"}:
            raise ValueError("block_table_pattern must be contiguous, shuffled or interleaved")
        batch, heads, seq_len, head_dim = (int(s) for s in k.shape)
        blocks_per_seq = (seq_len + block_size - 1) // block_size
        total = batch * blocks_per_seq
        perm = _layout_permutation(pattern, batch, blocks_per_seq, layout_seed, k.device)
        if perm is None:
            block_table = torch.arange(total, dtype=torch.int64, device=k.device).reshape(batch, blocks_per_seq)
        else:
            inverse = torch.empty_like(perm)
            inverse[perm] = torch.arange(total, dtype=torch.int64, device=k.device)
            block_table = inverse.reshape(batch, blocks_per_seq)

        if lengths is None:
            effective_lengths = torch.full((batch,), seq_len, dtype=torch.int64, device=k.device)
        else:
            effective_lengths = lengths.to(device=k.device, dtype=torch.int64).contiguous()
            if effective_lengths.ndim != 1 or effective_lengths.shape[0] != batch:
                raise ValueError("lengths must be [batch]")
            if bool((effective_lengths < 0).any().item()) or bool((effective_lengths > seq_len).any().item()):
                raise ValueError("lengths must lie in [0, seq_len]")

        if kv_format == "symmetric_token":
            k_quant = quantize_int8_symmetric_per_token(cls._physical_pages(k, block_size, perm))
            v_quant = quantize_int8_symmetric_per_token(cls._physical_pages(v, block_size, perm))
        elif kv_format == "affine_channel":
            if k.device.type == "cuda":
                k_quant = cls._quantize_pages(k, block_size, perm, total, per_channel=True)
                v_quant = cls._quantize_pages(v, block_size, perm, total, per_channel=True)
            else:
                k_quant = quantize_int8_per_channel(cls._physical_pages(k, block_size, perm), block_size=block_size)
                v_quant = quantize_int8_per_channel(cls._physical_pages(v, block_size, perm), block_size=block_size)
        elif kv_format == "fp8_block":
            if k.device.type == "cuda":
                k_quant = cls._quantize_pages(k, block_size, perm, total, fp8=True)
                v_quant = cls._quantize_pages(v, block_size, perm, total, fp8=True)
            else:
                k_quant = quantize_fp8_per_block(cls._physical_pages(k, block_size, perm), block_size=block_size)
                v_quant = quantize_fp8_per_block(cls._physical_pages(v, block_size, perm), block_size=block_size)
        elif k.device.type == "cuda":
            k_quant = cls._quantize_pages(k, block_size, perm, total)
            v_quant = cls._quantize_pages(v, block_size, perm, total)
        else:
            k_quant = quantize_int8_per_block(cls._physical_pages(k, block_size, perm), block_size=block_size)
            v_quant = quantize_int8_per_block(cls._physical_pages(v, block_size, perm), block_size=block_size)
        return cls(k_quant=k_quant, v_quant=v_quant, block_table=block_table, lengths=effective_lengths,
                   block_size=block_size, max_seq_len=seq_len)

    @staticmethod
    def _physical_pages(x: torch.Tensor, block_size: int, perm: torch.Tensor | None) -> torch.Tensor:
        batch, heads, seq_len, head_dim = x.shape
        n = (seq_len + block_size - 1) // block_size
        if n * block_size != seq_len:
            x = torch.cat([x, x.new_zeros((batch, heads, n * block_size - seq_len, head_dim))], dim=2)
        pages = (x.reshape(batch, heads, n, block_size, head_dim).permute(0, 2, 1, 3, 4).contiguous()
                 .reshape(batch * n, heads, block_size, head_dim))
        return pages if perm is None else pages[perm].contiguous()

    @staticmethod
    def _quantize_pages(x: torch.Tensor, block_size: int, perm: torch.Tensor | None, total: int,
                        fp8: bool = False, per_channel: bool = False) -> QuantizedTensor:
        lib = _lib.require()
        batch, heads, seq_len, head_dim = (int(s) for s in x.shape)
        src = _src_for_kernel(x.detach())
        values, scale, zero = _empty_page_store(total, heads, block_size, head_dim, x.device, per_channel)
        if fp8:
            values = values.view(FP8_DTYPE)
        page_src = None if perm is None else perm.to(torch.int64).contiguous()
        if fp8:
            quantize_pages = lib.fs_quantize_pages_fp8
        elif per_channel:
            quantize_pages = lib.fs_quantize_pages_i8_channel
        else:
            quantize_pages = lib.fs_quantize_pages_i8
        _lib.check(quantize_pages(
            src.data_ptr(), _lib.dtype_code(src.dtype), batch, heads, seq_len, head_dim, block_size,
            _lib.ptr(page_src), total, values.data_ptr(), scale.data_ptr(), zero.data_ptr(),
            _lib.stream_ptr(x.device)))
        return QuantizedTensor(values, scale, zero, block_size, (total, heads, block_size, head_dim))

    def to_dense(self) -> Tuple[torch.Tensor, torch.Tensor]:
        """Dequantize the store and gather ``[batch, heads, max_seq_len, dim]`` (paged.py:421-461)."""

        physical_k = dequantize_int8_per_block(self.k_quant, dtype=torch.float32)
        physical_v = dequantize_int8_per_block(self.v_quant, dtype=torch.float32)
        table = self.block_table.clamp_min(0)

        def gather(physical: torch.Tensor) -> torch.Tensor:
            return (physical[table].permute(0, 2, 1, 3, 4).contiguous()
                    .reshape(self.batch_size, self.num_heads, -1, self.head_dim)[..., : self.max_seq_len, :])

        return gather(physical_k), gather(physical_v)

    def append(self, k_new: torch.Tensor, v_new: torch.Tensor) -> "PagedKVCache":
        """Append ``[batch, heads, tokens, dim]`` to every row; returns a new cache (paged.py:463-557).

        Unallocated logical pages get fresh zero pages at the end of the store, and
        the whole store is requantized (block = page), as in the reference.
        """

        if is_fp8(self.k_quant) or is_fp8(self.v_quant) or is_per_channel(self.k_quant):
            raise ValueError("append requantizes pages in the reference's per-page affine INT8 format; FP8 and "
                             "per-channel caches are read-only")
        if k_new.ndim != 4 or v_new.ndim != 4:
            raise ValueError("k_new and v_new must be [batch, heads, tokens, head_dim]")
        if k_new.shape != v_new.shape:
            raise ValueError("k_new and v_new must have the same shape")
        if k_new.shape[0] != self.batch_size or k_new.shape[1] != self.num_heads or k_new.shape[3] != self.head_dim:
            raise ValueError("new KV batch, heads and head_dim must match the cache")
        tokens = int(k_new.shape[2])
        if tokens <= 0:
            raise ValueError("appended token dimension must be non-empty")
        if k_new.device != self.block_table.device or v_new.device != self.block_table.device:
            raise ValueError("new KV tensors must be on the cache's device")
        if self.block_table.device.type == "cuda":
            return self._append_hip(k_new, v_new, tokens)
        return self._append_portable(k_new, v_new, tokens)

    def _plan_append(self, tokens: int):
        bs = self.block_size
        table = self.block_table.detach().cpu().numpy().astype(np.int64, copy=True)
        lengths = self.lengths.detach().cpu().numpy().astype(np.int64, copy=True)
        required_cols = int(((lengths + tokens + bs - 1) // bs).max())
        if required_cols > table.shape[1]:
            table = np.concatenate(
                [table, np.full((table.shape[0], required_cols - table.shape[1]), -1, dtype=np.int64)], axis=1)
        return table, lengths

    def _append_hip(self, k_new: torch.Tensor, v_new: torch.Tensor, tokens: int) -> "PagedKVCache":
        bs, heads, dim = self.block_size, self.num_heads, self.head_dim
        in_pages = int(self.k_quant.original_shape[0])
        for q in (self.k_quant, self.v_quant):
            if tuple(q.original_shape) != (in_pages, heads, bs, dim):
                raise ValueError("PagedKVCache store must be [pages, heads, block_size, head_dim]")
        table, lengths = self._plan_append(tokens)
        writes = []
        next_page = in_pages
        for b in range(self.batch_size):
            start = int(lengths[b])
            for t in range(tokens):
                logical_block, offset = divmod(start + t, bs)
                phys = int(table[b, logical_block])
                if phys < 0:
                    phys = next_page
                    next_page += 1
                    table[b, logical_block] = phys
                writes.append((phys, offset, b * tokens + t))
        total = next_page
        row_src = np.full((total, bs), -1, dtype=np.int32)
        for phys, offset, src in writes:
            row_src[phys, offset] = src
        dev = k_new.device
        new_stores = []
        for q, src in ((self.k_quant, k_new), (self.v_quant, v_new)):
            out = _empty_page_store(total, heads, bs, dim, dev)
            _update_pages(q, out, None, total, None, row_src, src, heads=heads, page=bs, dim=dim)
            new_stores.append(QuantizedTensor(out[0], out[1], out[2], bs, (total, heads, bs, dim)))
        lengths = lengths + tokens
        return PagedKVCache(
            k_quant=new_stores[0], v_quant=new_stores[1],
            block_table=torch.from_numpy(table).to(dev), lengths=torch.from_numpy(lengths).to(dev),
            block_size=bs, max_seq_len=int(lengths.max()),
        )

    def _append_portable(self, k_new: torch.Tensor, v_new: torch.Tensor, tokens: int) -> "PagedKVCache":
        bs = self.block_size
        physical_k = dequantize_int8_per_block(self.k_quant, dtype=torch.float32).clone()
        physical_v = dequantize_int8_per_block(self.v_quant, dtype=torch.float32).clone()
        table_np, lengths_np = self._plan_append(tokens)
        k32 = k_new.to(dtype=torch.float32)
        v32 = v_new.to(dtype=torch.float32)
        zero_page = physical_k.new_zeros((1, self.num_heads, bs, self.head_dim))
        for b in range(self.batch_size):
            start = int(lengths_np[b])
            for t in range(tokens):
                logical_block, offset = divmod(start + t, bs)
                phys = int(table_np[b, logical_block])
                if phys < 0:  # a fresh zero page at the end of the store
                    phys = int(physical_k.shape[0])
                    physical_k = torch.cat([physical_k, zero_page])
                    physical_v = torch.cat([physical_v, zero_page])
                    table_np[b, logical_block] = phys
                physical_k[phys, :, offset, :] = k32[b, :, t, :]
                physical_v[phys, :, offset, :] = v32[b, :, t, :]
        lengths_np = lengths_np + tokens
        device = self.block_table.device
        return PagedKVCache(
            k_quant=quantize_int8_per_block(physical_k, block_size=bs),
            v_quant=quantize_int8_per_block(physical_v, block_size=bs),
            block_table=torch.from_numpy(table_np).to(device),
            lengths=torch.from_numpy(lengths_np).to(device),
            block_size=bs, max_seq_len=int(lengths_np.max()),
        )

    def estimated_bytes(self) -> int:
        """Quantized K/V stores + block_table + lengths (paged.py:559-577)."""

        table_bytes = self.block_table.numel() * self.block_table.element_size()
        length_bytes = self.lengths.numel() * self.lengths.element_size()
        return (estimate_quantized_bytes(self.k_quant) + estimate_quantized_bytes(self.v_quant)
                + table_bytes + length_bytes)
