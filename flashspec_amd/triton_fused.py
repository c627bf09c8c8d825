"""Kernel 1: contiguous INT8 KV decode attention on the HIP backend.

Drop-in for reference src/flashspec/triton_fused.py: same public entry
``fused_dequant_attention_triton(q, k_quant, v_quant, lengths=None,
return_stats=False)``, same private knob names, same validation errors.  The
launch goes to ``fs_fused_decode_i8`` (libflashspec_hip.so), which streams the
int8 K/V once, dequantizes in registers and merges split-K partials with an
fp32 log-sum-exp combine.
"""

from __future__ import annotations

import math
import weakref
from typing import Any

import torch

from . import _lib
from .quant import (FP8_DTYPE, QuantizedTensor, build_compression_stats, estimate_quantized_bytes, is_fp8,
                    is_per_channel)
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

__all__ = ["fused_dequant_attention_triton", "_compute_num_splits", "_resolve_block_n", "_resolve_num_warps"]

_DEFAULT_NUM_SPLITS = 4
_TOKENS_PER_SPLIT = 512
_S_MAX = 32


def _compute_num_splits(seq_len: int, block_n: int) -> int:
    """The reference's split-count rule (triton_fused.py:560-601), kept for its callers.

    ``FLASHSPEC_NUM_SPLITS`` wins (clamped to ``ceil(seq_len/block_n)``); otherwise
    1 split up to 512 tokens, else ``min(4, ceil(seq_len/block_n))`` capped at 32.
    The HIP launch sizes its splits for the GPU instead (``triton_utils.plan_splits``)
    and honours the same environment override.
    """

    from .triton_utils import forced_num_splits

    forced = forced_num_splits(seq_len, block_n)
    if forced is not None:
        return forced
    max_splits = max(1, (seq_len + block_n - 1) // block_n)
    if seq_len <= _TOKENS_PER_SPLIT:
        return 1
    return max(1, min(min(_DEFAULT_NUM_SPLITS, max_splits), _S_MAX))


def _validate_triton_fused_inputs(q: torch.Tensor, k_quant: QuantizedTensor, v_quant: QuantizedTensor,
                                  lengths: torch.Tensor | None) -> None:
    """Reference checks (triton_fused.py:506-548) plus the layout facts the kernel relies on."""

    validate_decode_query(q, kernel_name="fused")
    if len(k_quant.original_shape) != 4 or len(v_quant.original_shape) != 4:
        raise ValueError("k_quant and v_quant must come from [batch, heads, seq_len, head_dim] tensors")
    if k_quant.original_shape != v_quant.original_shape:
        raise ValueError("k_quant and v_quant original_shape must match")
    if tuple(q.shape) != (k_quant.original_shape[0], k_quant.original_shape[1], k_quant.original_shape[3]):
        raise ValueError("q batch, heads and head_dim must match the quantized K/V")
    if k_quant.device != q.device or v_quant.device != q.device:
        raise RuntimeError("q, k_quant and v_quant must be on the same GPU")
    if lengths is not None:
        if lengths.ndim != 1 or lengths.shape[0] != q.shape[0]:
            raise ValueError("lengths must be [batch]")
        if lengths.device != q.device:
            raise RuntimeError("lengths must be on q's GPU")
    if q.dtype not in _lib.DTYPE_CODE:
        raise ValueError("q dtype must be float16, bfloat16 or float32")
    batch, heads, seq_len, head_dim = k_quant.original_shape
    for name, qt in (("k_quant", k_quant), ("v_quant", v_quant)):
        if qt.values.dtype not in (torch.int8, FP8_DTYPE) or qt.scale.dtype != torch.float32 or \
                qt.zero_point.dtype != torch.int16:
            raise ValueError(f"{name} must hold int8 (or float8_e4m3fn) values, float32 scale and int16 zero_point")
        n_blocks = (seq_len + qt.block_size - 1) // qt.block_size
        if tuple(qt.values.shape) != (batch, heads, n_blocks, qt.block_size, head_dim):
            raise ValueError(f"{name}.values must be [batch, heads, n_blocks, block_size, head_dim]")
        per = head_dim if is_per_channel(qt) else 1
        if qt.scale.numel() != batch * heads * n_blocks * per or qt.zero_point.numel() != batch * heads * n_blocks * per:
            raise ValueError(f"{name} scale/zero_point must have one entry per block (or per block and channel)")
    if k_quant.block_size != v_quant.block_size:
        raise ValueError("K/V quant block sizes must match")
    if k_quant.values.dtype != v_quant.values.dtype or is_per_channel(k_quant) != is_per_channel(v_quant):
        raise ValueError("k_quant and v_quant must use the same format (int8 or float8_e4m3fn values, "
                         "per-block or per-channel scales)")
    if is_per_channel(k_quant) and is_fp8(k_quant):
        raise ValueError("per-channel scales are supported for INT8 stores")


def _run_fused_dequant_attention_triton(q: torch.Tensor, k_quant: QuantizedTensor, v_quant: QuantizedTensor,
                                        lengths: torch.Tensor | None = None, return_stats: bool = False,
                                        ) -> torch.Tensor | tuple[torch.Tensor, dict[str, float]]:
    """Launch the HIP fused kernel (replaces triton_fused.py:604-761); no dense K/V is built."""

    dev = q.device
    # the memo lives on k_quant; v_quant enters by identity (checked through a weak reference, so
    # a recycled id never matches), data pointer and element counts, lengths by shape, device
    # and dtype
    kv_, vv_ = k_quant.values, v_quant.values
    memo_key = (q.shape, q.dtype, dev, id(v_quant), kv_.data_ptr(), kv_.numel(), k_quant.scale.numel(),
                k_quant.zero_point.numel(), vv_.data_ptr(), vv_.numel(), v_quant.scale.numel(),
                v_quant.zero_point.numel(), None if lengths is None else (lengths.shape, lengths.device, lengths.dtype))
    memo = k_quant.__dict__.get("_fs_v_ref")
    if not (layout_checked(k_quant, memo_key) and memo is not None and memo() is v_quant):
        _validate_triton_fused_inputs(q, k_quant, v_quant, lengths)
        remember_layout(k_quant, memo_key)
        object.__setattr__(k_quant, "_fs_v_ref", weakref.ref(v_quant))
    lib = _lib.require()
    q_c = q.contiguous()
    kv = [t.contiguous() for t in (k_quant.values, k_quant.scale, k_quant.zero_point,
                                    v_quant.values, v_quant.scale, v_quant.zero_point)]
    lengths_c = None if lengths is None else lengths.to(torch.int64).contiguous()
    batch, heads, head_dim = (int(s) for s in q_c.shape)
    seq_len = int(k_quant.original_shape[-2])
    n_blocks = int(kv[0].shape[-3])
    block_size = int(k_quant.block_size)
    out = torch.empty_like(q_c)
    sm_scale = 1.0 / math.sqrt(float(head_dim))
    rows = batch * heads
    per_channel = is_per_channel(k_quant)
    light = q_c.dtype in (torch.float16, torch.bfloat16) and k_quant.values.dtype in (torch.int8, FP8_DTYPE)
    tiled, waves, split_tiles, max_splits, block_n = launch_plan(seq_len, rows, head_dim, block_size, block_size,
                                                                 dev, per_channel=per_channel, light=light,
                                                                 contiguous=True)
    stream = _lib.stream_ptr(dev)
    if tiled and max_splits > 1 and waves <= MERGE_MAX_WAVES:
        # split rows merge inside the decode launch (no workspace, no merge launch)
        area, area_bytes = merge_area(dev, rows, max_splits, head_dim, stream)
        _lib.check(lib.fs_fused_decode_merged(
            q_c.data_ptr(), _lib.dtype_code(q_c.dtype), kv_format_code(per_channel, is_fp8(k_quant)),
            *(t.data_ptr() for t in kv), _lib.ptr(lengths_c), out.data_ptr(), area.data_ptr(), area_bytes, batch,
            heads, head_dim, seq_len, n_blocks, block_size, sm_scale, split_tiles, max_splits, waves, stream))
        return _fused_result(out, return_stats, k_quant, v_quant, q_c, seq_len, max_splits, block_n, waves,
                             split_tiles, tiled)
    workspace, ws_bytes = None, 0
    if max_splits > 1:
        ws_bytes = int(lib.fs_decode_workspace_bytes(rows, max_splits, head_dim))
        workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
    if is_fp8(k_quant):
        _lib.check(lib.fs_fused_decode_fp8(
            q_c.data_ptr(), _lib.dtype_code(q_c.dtype), kv[0].data_ptr(), kv[1].data_ptr(), kv[3].data_ptr(),
            kv[4].data_ptr(), _lib.ptr(lengths_c), out.data_ptr(), _lib.ptr(workspace), ws_bytes, batch, heads,
            head_dim, seq_len, n_blocks, block_size, sm_scale, split_tiles, max_splits, waves, stream))
    else:
        decode = lib.fs_fused_decode_i8_channel if per_channel else lib.fs_fused_decode_i8
        _lib.check(decode(
            q_c.data_ptr(), _lib.dtype_code(q_c.dtype), *(t.data_ptr() for t in kv), _lib.ptr(lengths_c),
            out.data_ptr(), _lib.ptr(workspace), ws_bytes, batch, heads, head_dim, seq_len, n_blocks, block_size,
            sm_scale, split_tiles, max_splits, waves, stream))
    if max_splits > 1:
        _lib.check(lib.fs_combine_splits(
            workspace.data_ptr(), _lib.ptr(lengths_c), out.data_ptr(), _lib.dtype_code(out.dtype), batch, heads,
            head_dim, seq_len, split_tiles, max_splits, stream))
    return _fused_result(out, return_stats, k_quant, v_quant, q_c, seq_len, max_splits, block_n, waves, split_tiles,
                         tiled)


def _fused_result(out, return_stats, k_quant, v_quant, q_c, seq_len, max_splits, block_n, waves, split_tiles, tiled):
    """``out`` or ``(out, stats)`` with the reference's stats keys (triton_fused.py:746-761)."""

    if not return_stats:
        return out
    batch, heads, head_dim = (int(s) for s in q_c.shape)
    dense_bytes = 2 * batch * heads * seq_len * head_dim * q_c.element_size()
    quant_bytes = estimate_quantized_bytes(k_quant) + estimate_quantized_bytes(v_quant)
    return out, build_compression_stats(
        dense_bytes, quant_bytes, materializes_dense_kv=False,
        num_splits=float(max_splits), block_n=float(block_n), num_warps=float(waves),
        split_tiles=float(split_tiles), tiled_path=float(tiled),
    )


def fused_dequant_attention_triton(*_args: Any, **_kwargs: Any) -> Any:
    """Kernel 1 entry: HIP kernel for GPU tensors, portable ``fused_dequant_attention`` otherwise.

    Same signature as the reference (triton_fused.py:764-791):
    ``(q, k_quant, v_quant, lengths=None, return_stats=False)``.
    """

    def _load_fallback():
        from .attention import fused_dequant_attention

        return fused_dequant_attention

    return dispatch_triton_or_fallback(_args, _kwargs, run_triton=_run_fused_dequant_attention_triton,
                                       load_fallback=_load_fallback)
