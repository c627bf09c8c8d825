"""Affine per-block INT8 quantization (reference src/flashspec/quant.py), plus the symmetric
per-token INT8 and FP8 E4M3 per-block KV formats.

GPU tensors go to the HIP kernels of libflashspec_hip.so (``fs_quantize_i8``,
``fs_dequantize_i8``), whose float32 op sequence is bit-identical to the
reference's CPU result.  CPU tensors take the portable torch path, which is the
reference's own op sequence (quant.py:120-158).
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Tuple

import torch

from . import _lib


@dataclass(frozen=True)
class QuantizedTensor:
    """INT8 tensor quantized per ``[block_size, head_dim]`` block (quant.py:9-43).

    ``values`` int8 ``[..., n_blocks, block_size, head_dim]`` storing ``uint8 - 128``;
    ``scale`` fp32 and ``zero_point`` int16 (uint8 domain) ``[..., n_blocks, 1, 1]``;
    ``original_shape`` is the shape before sequence padding.
    """

    values: torch.Tensor
    scale: torch.Tensor
    zero_point: torch.Tensor
    block_size: int
    original_shape: Tuple[int, ...]

    @property
    def device(self) -> torch.device:
        return self.values.device


def _validate_block_tensor(x: torch.Tensor, block_size: int) -> None:
    """quant.py:46-66."""

    if x.ndim < 2:
        raise ValueError("input needs sequence and feature dimensions")
    if block_size <= 0:
        raise ValueError("block_size must be positive")
    if x.shape[-1] <= 0 or x.shape[-2] <= 0:
        raise ValueError("sequence and feature dimensions must be non-empty")


def _pad_sequence_dim(x: torch.Tensor, block_size: int) -> torch.Tensor:
    """Zero-pad dim -2 up to a multiple of block_size (quant.py:69-91)."""

    pad = (block_size - x.shape[-2] % block_size) % block_size
    if pad == 0:
        return x
    return torch.cat([x, x.new_zeros((*x.shape[:-2], pad, x.shape[-1]))], dim=-2)


def _quantize_portable(x: torch.Tensor, block_size: int) -> QuantizedTensor:
    original_shape = tuple(x.shape)
    xf = _pad_sequence_dim(x.detach().to(torch.float32), block_size)
    lead, seq, dim = xf.shape[:-2], xf.shape[-2], xf.shape[-1]
    blocked = xf.reshape(*lead, seq // block_size, block_size, dim)
    lo = blocked.amin(dim=(-2, -1), keepdim=True)
    hi = blocked.amax(dim=(-2, -1), keepdim=True)
    scale = ((hi - lo) / 255.0).clamp_min(1.0e-8)
    zero = torch.round(-lo / scale).clamp(0, 255)
    codes = torch.round(blocked / scale + zero).clamp(0, 255)
    values = (codes.to(torch.int16) - 128).to(torch.int8)
    return QuantizedTensor(values, scale, zero.to(torch.int16), block_size, original_shape)


def _quantize_hip(x: torch.Tensor, block_size: int) -> QuantizedTensor:
    lib = _lib.require()
    original_shape = tuple(x.shape)
    xd = x.detach()
    if xd.dtype not in _lib.DTYPE_CODE:
        xd = xd.to(torch.float32)
    xd = xd.contiguous()
    lead = tuple(xd.shape[:-2])
    seq, dim = int(xd.shape[-2]), int(xd.shape[-1])
    n_blocks = (seq + block_size - 1) // block_size
    outer = math.prod(lead) if lead else 1
    dev = xd.device
    values = torch.empty((*lead, n_blocks, block_size, dim), dtype=torch.int8, device=dev)
    scale = torch.empty((*lead, n_blocks, 1, 1), dtype=torch.float32, device=dev)
    zero = torch.empty((*lead, n_blocks, 1, 1), dtype=torch.int16, device=dev)
    if outer > 0:
        _lib.check(lib.fs_quantize_i8(
            xd.data_ptr(), _lib.dtype_code(xd.dtype), outer, seq, dim, block_size,
            values.data_ptr(), scale.data_ptr(), zero.data_ptr(), _lib.stream_ptr(dev)))
    return QuantizedTensor(values, scale, zero, block_size, original_shape)


def quantize_int8_per_block(x: torch.Tensor, block_size: int = 16) -> QuantizedTensor:
    """Affine INT8 quantization of ``x`` per ``[block_size, head_dim]`` block (quant.py:94-165).

    The zero padding of a ragged last block takes part in its min/max.
    """

    _validate_block_tensor(x, block_size)
    if x.device.type == "cuda":
        return _quantize_hip(x, block_size)
    return _quantize_portable(x, block_size)


def _quantize_sym_portable(x: torch.Tensor) -> QuantizedTensor:
    xf = x.detach().to(torch.float32)
    lead, seq, dim = tuple(xf.shape[:-2]), xf.shape[-2], xf.shape[-1]
    scale = (xf.abs().amax(dim=-1, keepdim=True) / 127.0).clamp_min(1.0e-8)
    codes = torch.round(xf / scale).clamp(-127, 127).to(torch.int8)
    zero = torch.full((*lead, seq, 1, 1), 128, dtype=torch.int16, device=xf.device)
    return QuantizedTensor(codes.reshape(*lead, seq, 1, dim), scale.reshape(*lead, seq, 1, 1), zero, 1,
                           tuple(x.shape))


def _quantize_sym_hip(x: torch.Tensor) -> QuantizedTensor:
    lib = _lib.require()
    xd = x.detach()
    if xd.dtype not in _lib.DTYPE_CODE:
        xd = xd.to(torch.float32)
    xd = xd.contiguous()
    lead, seq, dim = tuple(xd.shape[:-2]), int(xd.shape[-2]), int(xd.shape[-1])
    rows = math.prod(lead) * seq if lead else seq
    dev = xd.device
    values = torch.empty((*lead, seq, 1, dim), dtype=torch.int8, device=dev)
    scale = torch.empty((*lead, seq, 1, 1), dtype=torch.float32, device=dev)
    zero = torch.empty((*lead, seq, 1, 1), dtype=torch.int16, device=dev)
    if rows > 0:
        _lib.check(lib.fs_quantize_sym_i8(xd.data_ptr(), _lib.dtype_code(xd.dtype), rows, dim, values.data_ptr(),
                                          scale.data_ptr(), zero.data_ptr(), _lib.stream_ptr(dev)))
    return QuantizedTensor(values, scale, zero, 1, tuple(x.shape))


def quantize_int8_symmetric_per_token(x: torch.Tensor) -> QuantizedTensor:
    """Symmetric absmax INT8 with one fp32 scale per token row (per head).

    ``scale = max(absmax(row) / 127, 1e-8)``, ``q = clamp(round(x / scale), -127, 127)``.
    Not in the reference (its quantizer is ``quantize_int8_per_block``); returned in the
    same affine layout with ``block_size = 1`` and zero point 128, so ``dequantize_int8_per_block``,
    the portable attention paths and the HIP decode kernels all read it unchanged.
    """

    _validate_block_tensor(x, 1)
    if x.device.type == "cuda":
        return _quantize_sym_hip(x)
    return _quantize_sym_portable(x)


# ---- per-channel affine INT8 -----------------------------------------------------------------
# A KV format beside the reference's (which lists per-channel scales among the formats to
# compare, doc/TODO.MD:241-255): the reference's per-block op sequence applied to each channel
# column of a block, so scale / zero_point are [..., n_blocks, 1, head_dim] and every
# dequantize formula here broadcasts over them unchanged.


def is_per_channel(q: QuantizedTensor) -> bool:
    """True when scale / zero_point hold one entry per channel of each block."""

    return q.values.shape[-1] > 1 and q.scale.shape[-1] == q.values.shape[-1]


def _quantize_channel_portable(x: torch.Tensor, block_size: int) -> QuantizedTensor:
    original_shape = tuple(x.shape)
    xf = _pad_sequence_dim(x.detach().to(torch.float32), block_size)
    lead, seq, dim = xf.shape[:-2], xf.shape[-2], xf.shape[-1]
    blocked = xf.reshape(*lead, seq // block_size, block_size, dim)
    lo = blocked.amin(dim=-2, keepdim=True)
    hi = blocked.amax(dim=-2, keepdim=True)
    scale = ((hi - lo) / 255.0).clamp_min(1.0e-8)
    zero = torch.round(-lo / scale).clamp(0, 255)
    codes = torch.round(blocked / scale + zero).clamp(0, 255)
    values = (codes.to(torch.int16) - 128).to(torch.int8)
    return QuantizedTensor(values, scale, zero.to(torch.int16), block_size, original_shape)


def _quantize_channel_hip(x: torch.Tensor, block_size: int) -> QuantizedTensor:
    lib = _lib.require()
    original_shape = tuple(x.shape)
    xd = x.detach()
    if xd.dtype not in _lib.DTYPE_CODE:
        xd = xd.to(torch.float32)
    xd = xd.contiguous()
    lead = tuple(xd.shape[:-2])
    seq, dim = int(xd.shape[-2]), int(xd.shape[-1])
    n_blocks = (seq + block_size - 1) // block_size
    outer = math.prod(lead) if lead else 1
    dev = xd.device
    values = torch.empty((*lead, n_blocks, block_size, dim), dtype=torch.int8, device=dev)
    scale = torch.empty((*lead, n_blocks, 1, dim), dtype=torch.float32, device=dev)
    zero = torch.empty((*lead, n_blocks, 1, dim), dtype=torch.int16, device=dev)
    if outer > 0:
        _lib.check(lib.fs_quantize_i8_channel(
            xd.data_ptr(), _lib.dtype_code(xd.dtype), outer, seq, dim, block_size,
            values.data_ptr(), scale.data_ptr(), zero.data_ptr(), _lib.stream_ptr(dev)))
    return QuantizedTensor(values, scale, zero, block_size, original_shape)


def quantize_int8_per_channel(x: torch.Tensor, block_size: int = 16) -> QuantizedTensor:
    """Affine INT8 with one scale / zero point per ``block_size`` tokens and per channel.

    Each channel column of a block is quantized as ``quantize_int8_per_block`` would quantize
    that ``[block_size, 1]`` column; ``scale`` / ``zero_point`` are ``[..., n_blocks, 1, D]``.
    The decode kernels read it with quant blocks of a multiple of 16 tokens (other shapes run
    the element-wise kernel).
    """

    _validate_block_tensor(x, block_size)
    if x.device.type == "cuda":
        return _quantize_channel_hip(x, block_size)
    return _quantize_channel_portable(x, block_size)


# ---- FP8 E4M3 per-block format ----------------------------------------------------------------
# A KV format beside the reference's (which lists FP8 among the formats to compare,
# doc/TODO.MD:241-255): OCP FP8 E4M3 codes (torch.float8_e4m3fn) in the same block layout, one
# fp32 scale per block and no zero point (the zero_point tensor is all 0):
#     scale = max(absmax / 448, 1e-8);  code = E4M3_RNE(clamp(x / scale, -448, 448))
# gfx950 converts natively (v_cvt_pk_fp8_f32 / v_cvt_pk_f32_fp8), rounding like torch's cast.

FP8_DTYPE = torch.float8_e4m3fn
FP8_MAX = 448.0


def is_fp8(q: QuantizedTensor) -> bool:
    """True for the FP8 E4M3 format (values of dtype float8_e4m3fn)."""

    return q.values.dtype == FP8_DTYPE


def _quantize_fp8_portable(x: torch.Tensor, block_size: int) -> QuantizedTensor:
    original_shape = tuple(x.shape)
    xf = _pad_sequence_dim(x.detach().to(torch.float32), block_size)
    lead, seq, dim = xf.shape[:-2], xf.shape[-2], xf.shape[-1]
    blocked = xf.reshape(*lead, seq // block_size, block_size, dim)
    scale = (blocked.abs().amax(dim=(-2, -1), keepdim=True) / FP8_MAX).clamp_min(1.0e-8)
    codes = (blocked / scale).clamp(-FP8_MAX, FP8_MAX).to(FP8_DTYPE)
    return QuantizedTensor(codes, scale, torch.zeros_like(scale, dtype=torch.int16), block_size, original_shape)


def _quantize_fp8_hip(x: torch.Tensor, block_size: int) -> QuantizedTensor:
    lib = _lib.require()
    original_shape = tuple(x.shape)
    xd = x.detach()
    if xd.dtype not in _lib.DTYPE_CODE:
        xd = xd.to(torch.float32)
    xd = xd.contiguous()
    lead = tuple(xd.shape[:-2])
    seq, dim = int(xd.shape[-2]), int(xd.shape[-1])
    n_blocks = (seq + block_size - 1) // block_size
    outer = math.prod(lead) if lead else 1
    dev = xd.device
    values = torch.empty((*lead, n_blocks, block_size, dim), dtype=FP8_DTYPE, device=dev)
    scale = torch.empty((*lead, n_blocks, 1, 1), dtype=torch.float32, device=dev)
    zero = torch.empty((*lead, n_blocks, 1, 1), dtype=torch.int16, device=dev)
    if outer > 0:
        _lib.check(lib.fs_quantize_fp8(
            xd.data_ptr(), _lib.dtype_code(xd.dtype), outer, seq, dim, block_size,
            values.data_ptr(), scale.data_ptr(), zero.data_ptr(), _lib.stream_ptr(dev)))
    return QuantizedTensor(values, scale, zero, block_size, original_shape)


def quantize_fp8_per_block(x: torch.Tensor, block_size: int = 16) -> QuantizedTensor:
    """FP8 E4M3 quantization of ``x`` per ``[block_size, head_dim]`` block, one fp32 scale each.

    Same layout and padding as ``quantize_int8_per_block``; ``values`` are float8_e4m3fn codes
    and ``zero_point`` is all zero.  Every attention entry point and ``dequantize_int8_per_block``
    read it.
    """

    _validate_block_tensor(x, block_size)
    if x.device.type == "cuda":
        return _quantize_fp8_hip(x, block_size)
    return _quantize_fp8_portable(x, block_size)


def _dequantize_fp8(q: QuantizedTensor, dtype: torch.dtype | None) -> torch.Tensor:
    lead = tuple(q.original_shape[:-2])
    seq, dim = int(q.original_shape[-2]), int(q.original_shape[-1])
    if q.values.device.type != "cuda":
        x = q.values.to(torch.float32) * q.scale.to(torch.float32)
        x = x.reshape(*lead, -1, dim)[..., :seq, :]
        return x.to(dtype=dtype) if dtype is not None else x
    lib = _lib.require()
    values = q.values.contiguous()
    n_blocks, block = int(values.shape[-3]), int(values.shape[-2])
    outer = values.numel() // max(1, n_blocks * block * dim)
    out_dtype = dtype if dtype in _lib.DTYPE_CODE else torch.float32
    out = torch.empty((*lead, seq, dim), dtype=out_dtype, device=values.device)
    if out.numel() > 0:
        scale = q.scale.to(torch.float32).contiguous()
        if scale.numel() != outer * n_blocks:
            raise ValueError("scale does not match the quantized values' block count")
        _lib.check(lib.fs_dequantize_fp8(
            values.data_ptr(), scale.data_ptr(), outer, n_blocks, block, dim, seq,
            out.data_ptr(), _lib.dtype_code(out_dtype), _lib.stream_ptr(values.device)))
    if dtype is not None and dtype != out_dtype:
        out = out.to(dtype)
    return out


def _dequantize_hip(q: QuantizedTensor, dtype: torch.dtype | None) -> torch.Tensor:
    lib = _lib.require()
    lead = tuple(q.original_shape[:-2])
    seq, dim = int(q.original_shape[-2]), int(q.original_shape[-1])
    values = q.values.contiguous()
    n_blocks, block = int(values.shape[-3]), int(values.shape[-2])
    outer = values.numel() // max(1, n_blocks * block * dim)
    out_dtype = dtype if dtype in _lib.DTYPE_CODE else torch.float32
    out = torch.empty((*lead, seq, dim), dtype=out_dtype, device=values.device)
    if out.numel() > 0:
        scale = q.scale.to(torch.float32).contiguous()
        zero = q.zero_point.to(torch.int16).contiguous()
        if scale.numel() != outer * n_blocks or zero.numel() != outer * n_blocks:
            raise ValueError("scale/zero_point do not match the quantized values' block count")
        _lib.check(lib.fs_dequantize_i8(
            values.data_ptr(), scale.data_ptr(), zero.data_ptr(), outer, n_blocks, block, dim, seq,
            out.data_ptr(), _lib.dtype_code(out_dtype), _lib.stream_ptr(values.device)))
    if dtype is not None and dtype != out_dtype:
        out = out.to(dtype)
    return out


def dequantize_int8_per_block(q: QuantizedTensor, dtype: torch.dtype | None = None) -> torch.Tensor:
    """``((values + 128) - zero_point) * scale``, padding cropped (quant.py:168-204); for the
    FP8 format (``is_fp8``) ``float(code) * scale``."""

    if is_fp8(q):
        return _dequantize_fp8(q, dtype)
    if q.values.device.type == "cuda" and not is_per_channel(q):
        return _dequantize_hip(q, dtype)
    u = q.values.to(torch.int16) + 128
    x = (u.to(torch.float32) - q.zero_point.to(torch.float32)) * q.scale.to(torch.float32)
    lead, seq, dim = q.original_shape[:-2], q.original_shape[-2], q.original_shape[-1]
    x = x.reshape(*lead, -1, dim)[..., :seq, :]
    return x.to(dtype=dtype) if dtype is not None else x


def build_compression_stats(dense_bytes: float, quant_bytes: float, *, materializes_dense_kv: bool,
                            **extra: float) -> dict[str, float]:
    """Stats dict shared by every attention path (quant.py:207-229)."""

    stats = {
        "dense_kv_bytes": float(dense_bytes),
        "quant_kv_bytes": float(quant_bytes),
        "compression_ratio": float(dense_bytes / max(1, quant_bytes)),
        "materializes_dense_kv": 1.0 if materializes_dense_kv else 0.0,
    }
    stats.update({key: float(value) for key, value in extra.items()})
    return stats


def dequantize_fp8_per_block(q: QuantizedTensor, dtype: torch.dtype | None = None) -> torch.Tensor:
    """``float(code) * scale`` of an FP8 E4M3 ``QuantizedTensor``, padding cropped."""

    if not is_fp8(q):
        raise ValueError("dequantize_fp8_per_block takes the FP8 E4M3 format (float8_e4m3fn values)")
    return _dequantize_fp8(q, dtype)


def estimate_quantized_bytes(q: QuantizedTensor) -> int:
    """int8 values + 4 B per scale + 2 B per zero point (quant.py:232-247)."""

    return q.values.numel() + q.scale.numel() * 4 + q.zero_point.numel() * 2
