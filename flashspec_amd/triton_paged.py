"""Kernel 2: paged INT8 KV decode attention on the HIP backend.

Drop-in for reference src/flashspec/triton_paged.py: same public entry
``paged_quant_attention_triton(q, cache, return_stats=False)``, same knob names
and validation errors.  The launch goes to ``fs_paged_decode_i8``: a workgroup of
cooperating waves resolves each block_table entry once per page into a base offset
(instead of per-token-lane table loads), streams the int8 pages with coalesced
16-byte loads and merges its waves in LDS; rows only split across workgroups when
there are fewer rows than CUs, and then the last split of each row to finish merges
the row (fp32 log-sum-exp) inside the same launch (``fs_paged_decode_merged``).
"""

from __future__ import annotations

import math
from typing import Any

import torch

from . import _lib
from .paged import PagedKVCache
from .quant import FP8_DTYPE, build_compression_stats, is_fp8, is_per_channel
from .triton_utils import (
    dispatch_triton_or_fallback,
    MERGE_MAX_WAVES,
    kv_format_code,
    launch_plan,
    layout_checked,
    merge_area,
    remember_layout,
    resolve_block_n as _resolve_block_n,
    resolve_num_warps as _resolve_num_warps,
    validate_decode_query,
)

__all__ = ["paged_quant_attention_triton", "_resolve_block_n", "_resolve_num_warps"]


def _validate_triton_paged_inputs(q: torch.Tensor, cache: PagedKVCache) -> None:
    """Reference checks (triton_paged.py:302-335) plus the layout facts the kernel relies on."""

    validate_decode_query(q, kernel_name="paged")
    if q.shape[0] != cache.batch_size or q.shape[1] != cache.num_heads or q.shape[2] != cache.head_dim:
        raise ValueError("q batch, heads and head_dim must match the PagedKVCache")
    if cache.k_quant.original_shape != cache.v_quant.original_shape:
        raise ValueError("cache.k_quant and cache.v_quant original_shape must match")
    if len(cache.k_quant.original_shape) != 4:
        raise ValueError("PagedKVCache k_quant/v_quant must come from [physical, heads, block, head_dim] tensors")
    if cache.k_quant.original_shape[2] != cache.block_size:
        raise ValueError("the physical page's sequence dim must equal cache.block_size")
    if cache.k_quant.block_size != cache.v_quant.block_size:
        raise ValueError("K/V quant block_size must match")
    if cache.block_size % cache.k_quant.block_size != 0:
        raise ValueError("cache.block_size must be a multiple of the quant block_size")
    if cache.k_quant.device != q.device or cache.v_quant.device != q.device:
        raise RuntimeError("q and the cache's quantized K/V must be on the same GPU")
    if cache.block_table.device != q.device or cache.lengths.device != q.device:
        raise RuntimeError("block_table and lengths must be on q's GPU")
    if q.dtype not in _lib.DTYPE_CODE:
        raise ValueError("q dtype must be float16, bfloat16 or float32")
    pages, heads, page, head_dim = cache.k_quant.original_shape
    qb = cache.k_quant.block_size
    if cache.k_quant.values.dtype != cache.v_quant.values.dtype or \
            is_per_channel(cache.k_quant) != is_per_channel(cache.v_quant):
        raise ValueError("cache K and V must use the same format (int8 or float8_e4m3fn values, per-block or "
                         "per-channel scales)")
    if is_per_channel(cache.k_quant) and is_fp8(cache.k_quant):
        raise ValueError("per-channel scales are supported for INT8 stores")
    for name, qt in (("k_quant", cache.k_quant), ("v_quant", cache.v_quant)):
        if qt.values.dtype not in (torch.int8, FP8_DTYPE) or qt.scale.dtype != torch.float32 or \
                qt.zero_point.dtype != torch.int16:
            raise ValueError(f"cache.{name} must hold int8 (or float8_e4m3fn) values, float32 scale and int16 "
                             "zero_point")
        if tuple(qt.values.shape) != (pages, heads, page // qb, qb, head_dim):
            raise ValueError(f"cache.{name}.values must be [pages, heads, page/quant_block, quant_block, head_dim]")
        per = head_dim if is_per_channel(qt) else 1
        n_params = pages * heads * (page // qb) * per
        if qt.scale.numel() != n_params or qt.zero_point.numel() != n_params:
            raise ValueError(f"cache.{name} scale/zero_point must have one entry per quant block (or per block and "
                             "channel)")
    if cache.block_table.ndim != 2 or cache.block_table.dtype not in (torch.int32, torch.int64):
        raise ValueError("block_table must be a 2-D int32/int64 tensor")
    if cache.lengths.ndim != 1 or cache.lengths.shape[0] != cache.batch_size:
        raise ValueError("lengths must be [batch]")


def _run_paged_quant_attention_triton(q: torch.Tensor, cache: PagedKVCache, return_stats: bool = False,
                                      request_order: torch.Tensor | None = None,
                                      ) -> torch.Tensor | tuple[torch.Tensor, dict[str, float]]:
    """Launch the HIP paged kernel (replaces triton_paged.py:338-450); no dense K/V is built.

    ``request_order`` (device int32 permutation of the batch, affine INT8 stores on the tiled path):
    dispatch the requests in that order (``fs_paged_decode_ordered``); the output is the same."""

    kq, vq = cache.k_quant, cache.v_quant
    dev = q.device
    table, lens = cache.block_table, cache.lengths
    memo_key = (q.shape, q.dtype, dev, table.data_ptr(), table.numel(), lens.data_ptr(), lens.numel(),
                kq.values.data_ptr(), kq.values.numel(), kq.scale.numel(), kq.zero_point.numel(),
                vq.values.data_ptr(), vq.values.numel(), vq.scale.numel(), vq.zero_point.numel())
    if not layout_checked(cache, memo_key):
        _validate_triton_paged_inputs(q, cache)
        remember_layout(cache, memo_key)
    lib = _lib.require()
    q_c = q.contiguous()
    kv = [t.contiguous() for t in (kq.values, kq.scale, kq.zero_point, vq.values, vq.scale, vq.zero_point)]
    table = cache.block_table.contiguous()
    lengths = cache.lengths if cache.lengths.dtype == torch.int64 else cache.lengths.to(torch.int64)
    lengths = lengths.contiguous()
    batch, heads, head_dim = (int(s) for s in q_c.shape)
    max_seq_len = int(cache.max_seq_len)
    num_pages = int(kq.original_shape[0])
    out = torch.empty_like(q_c)
    sm_scale = 1.0 / math.sqrt(float(head_dim))
    rows = batch * heads
    per_channel = is_per_channel(kq)
    light = q_c.dtype in (torch.float16, torch.bfloat16) and kq.values.dtype in (torch.int8, FP8_DTYPE)
    tiled, waves, split_tiles, max_splits, block_n = launch_plan(
        max_seq_len, rows, head_dim, int(cache.block_size), int(kq.block_size), dev, per_channel=per_channel,
        light=light)
    stream = _lib.stream_ptr(dev)
    if request_order is not None and tiled and not per_channel and not is_fp8(kq):
        area, area_bytes, workspace, ws_bytes = None, 0, None, 0
        if max_splits > 1 and waves <= MERGE_MAX_WAVES:
            area, area_bytes = merge_area(dev, rows, max_splits, head_dim, stream)
        elif max_splits > 1:
            ws_bytes = int(lib.fs_decode_workspace_bytes(rows, max_splits, head_dim))
            workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        _lib.check(lib.fs_paged_decode_ordered(
            q_c.data_ptr(), _lib.dtype_code(q_c.dtype), *(t.data_ptr() for t in kv), table.data_ptr(),
            table.element_size(), int(table.shape[1]), lengths.data_ptr(), request_order.data_ptr(), out.data_ptr(),
            _lib.ptr(workspace), ws_bytes, _lib.ptr(area), area_bytes, batch, heads, head_dim, num_pages,
            int(cache.block_size), int(kq.block_size), max_seq_len, sm_scale, split_tiles, max_splits, waves, stream))
        return _paged_result(out, return_stats, cache, q_c, max_seq_len, max_splits, block_n, waves, split_tiles,
                             tiled)
    if tiled and max_splits > 1 and waves <= MERGE_MAX_WAVES:
        # split rows merge inside the decode launch (no workspace, no merge launch)
        area, area_bytes = merge_area(dev, rows, max_splits, head_dim, stream)
        _lib.check(lib.fs_paged_decode_merged(
            q_c.data_ptr(), _lib.dtype_code(q_c.dtype), kv_format_code(per_channel, is_fp8(kq)),
            *(t.data_ptr() for t in kv), table.data_ptr(), table.element_size(), int(table.shape[1]),
            lengths.data_ptr(), out.data_ptr(), area.data_ptr(), area_bytes, batch, heads, head_dim, num_pages,
            int(cache.block_size), int(kq.block_size), max_seq_len, sm_scale, split_tiles, max_splits, waves, stream))
        return _paged_result(out, return_stats, cache, q_c, max_seq_len, max_splits, block_n, waves, split_tiles,
                             tiled)
    workspace, ws_bytes = None, 0
    if max_splits > 1:
        ws_bytes = int(lib.fs_decode_workspace_bytes(rows, max_splits, head_dim))
        workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    if is_fp8(kq):
        _lib.check(lib.fs_paged_decode_fp8(
            q_c.data_ptr(), _lib.dtype_code(q_c.dtype), kv[0].data_ptr(), kv[1].data_ptr(), kv[3].data_ptr(),
            kv[4].data_ptr(), table.data_ptr(), table.element_size(), int(table.shape[1]), lengths.data_ptr(),
            out.data_ptr(), _lib.ptr(workspace), ws_bytes, batch, heads, head_dim, num_pages, int(cache.block_size),
            int(kq.block_size), max_seq_len, sm_scale, split_tiles, max_splits, waves, stream))
    else:
        decode = lib.fs_paged_decode_i8_channel if per_channel else lib.fs_paged_decode_i8
        _lib.check(decode(
            q_c.data_ptr(), _lib.dtype_code(q_c.dtype), *(t.data_ptr() for t in kv), table.data_ptr(),
            table.element_size(), int(table.shape[1]), lengths.data_ptr(), out.data_ptr(), _lib.ptr(workspace),
            ws_bytes, batch, heads, head_dim, num_pages, int(cache.block_size), int(kq.block_size), max_seq_len,
            sm_scale, split_tiles, max_splits, waves, stream))
    if max_splits > 1:
        _lib.check(lib.fs_combine_splits(
            workspace.data_ptr(), lengths.data_ptr(), out.data_ptr(), _lib.dtype_code(out.dtype), batch, heads,
            head_dim, max_seq_len, split_tiles, max_splits, stream))
    return _paged_result(out, return_stats, cache, q_c, max_seq_len, max_splits, block_n, waves, split_tiles, tiled)


def _paged_result(out, return_stats, cache, q_c, max_seq_len, max_splits, block_n, waves, split_tiles, tiled):
    """``out`` or ``(out, stats)`` with the reference's stats keys (triton_paged.py:439-449)."""

    if not return_stats:
        return out
    batch, heads, head_dim = (int(s) for s in q_c.shape)
    dense_bytes = 2 * batch * heads * max_seq_len * head_dim * q_c.element_size()
    return out, build_compression_stats(
        dense_bytes, cache.estimated_bytes(), materializes_dense_kv=False,
        physical_blocks=float(cache.block_table.ge(0).sum().item()),
        block_n=float(block_n), num_warps=float(waves), num_splits=float(max_splits),
        split_tiles=float(split_tiles), tiled_path=float(tiled),
    )


def paged_quant_attention_triton(*_args: Any, **_kwargs: Any) -> Any:
    """Kernel 2 entry: HIP kernel for a GPU ``q`` with a ``PagedKVCache``, portable path otherwise.

    Same signature as the reference (triton_paged.py:453-490): ``(q, cache, return_stats=False)``.
    """

    def _needs_paged_cache(args) -> bool:
        return len(args) >= 2 and isinstance(args[1], PagedKVCache)

    def _load_fallback():
        from .attention import paged_quant_attention

        return paged_quant_attention

    return dispatch_triton_or_fallback(_args, _kwargs, run_triton=_run_paged_quant_attention_triton,
                                       load_fallback=_load_fallback, extra_guard=_needs_paged_cache)
