"""Oracle: affine per-block INT8 quantization (test infrastructure only).

Restates reference src/flashspec/quant.py:94-204 in numpy float32.  Every torch
op there is one IEEE-754 float32 operation, so the same op sequence in numpy
float32 gives the same bits:

* ``(mx - mn) / 255.0``       -> float32 subtraction, float32 true division
* ``clamp_min(1e-8)``         -> max with float32(1e-8)
* ``round(-mn / scale)``      -> float32 division, round-half-to-even
* ``round(x / scale + zp)``   -> float32 division, float32 add, half-to-even
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Tuple

import numpy as np

F32 = np.float32
SCALE_FLOOR = F32(1.0e-8)


@dataclass(frozen=True)
class OracleQuant:
    """Mirror of ``QuantizedTensor`` (reference quant.py:9-41)."""

    values: np.ndarray  # int8 [..., n_blocks, block_size, head_dim]
    scale: np.ndarray  # float32 [..., n_blocks, 1, 1]
    zero_point: np.ndarray  # int16 [..., n_blocks, 1, 1]
    block_size: int
    original_shape: Tuple[int, ...]


def pad_sequence_dim(x: np.ndarray, block_size: int) -> np.ndarray:
    """Zero-pad the sequence axis (-2) up to a multiple of block_size (quant.py:69-91)."""

    pad = (-x.shape[-2]) % block_size
    if pad == 0:
        return x
    widths = [(0, 0)] * x.ndim
    widths[-2] = (0, pad)
    return np.pad(x, widths)


def quantize_int8_per_block(x: np.ndarray, block_size: int = 16) -> OracleQuant:
    """Affine INT8 quantization per [block_size, head_dim] block (quant.py:94-165).

    The zero padding of a ragged tail block takes part in min/max (quant.py:120).
    """

    if x.ndim < 2:
        raise ValueError("x needs sequence and feature axes")
    if block_size <= 0:
        raise ValueError("block_size must be positive")
    if x.shape[-1] <= 0 or x.shape[-2] <= 0:
        raise ValueError("sequence and feature axes must be non-empty")
    original_shape = tuple(int(s) for s in x.shape)
    xf = pad_sequence_dim(np.asarray(x).astype(F32), block_size)
    lead = xf.shape[:-2]
    n_blocks = xf.shape[-2] // block_size
    blocked = xf.reshape(*lead, n_blocks, block_size, xf.shape[-1])
    mn = blocked.min(axis=(-2, -1), keepdims=True)
    mx = blocked.max(axis=(-2, -1), keepdims=True)
    scale = np.maximum((mx - mn) / F32(255.0), SCALE_FLOOR).astype(F32)  # quant.py:146
    zp = np.clip(np.rint(-mn / scale), F32(0), F32(255)).astype(F32)  # quant.py:150
    qu = np.clip(np.rint(blocked / scale + zp), F32(0), F32(255))  # quant.py:154
    values = (qu.astype(np.int16) - 128).astype(np.int8)  # quant.py:158
    return OracleQuant(values, scale, zp.astype(np.int16), block_size, original_shape)


def dequantize_int8_per_block(q: OracleQuant) -> np.ndarray:
    """``(float(v + 128) - float(zp)) * scale``, then crop the padding (quant.py:168-204)."""

    u = q.values.astype(np.int16) + 128
    x = (u.astype(F32) - q.zero_point.astype(F32)) * q.scale.astype(F32)
    lead = q.original_shape[:-2]
    seq_len, head_dim = q.original_shape[-2], q.original_shape[-1]
    return x.reshape(*lead, -1, head_dim)[..., :seq_len, :].astype(F32)


def quantize_int8_per_channel(x: np.ndarray, block_size: int = 16) -> OracleQuant:
    """Affine INT8 with one scale / zero point per block of ``block_size`` tokens and per
    channel: a KV format offered beside the reference's (which lists per-channel scales among
    the formats to compare, doc/TODO.MD:241-255).  Each channel column of a block is quantized
    exactly as the reference's per-block quantizer would quantize that [block_size, 1] column
    (same float32 op sequence, padding included), which tests/test_oracle.py checks; scale and
    zero_point are [..., n_blocks, 1, head_dim], so dequantize_int8_per_block's broadcast formula
    reads it unchanged.
    """

    if x.ndim < 2:
        raise ValueError("x needs sequence and feature axes")
    if block_size <= 0:
        raise ValueError("block_size must be positive")
    if x.shape[-1] <= 0 or x.shape[-2] <= 0:
        raise ValueError("sequence and feature axes must be non-empty")
    original_shape = tuple(int(s) for s in x.shape)
    xf = pad_sequence_dim(np.asarray(x).astype(F32), block_size)
    lead = xf.shape[:-2]
    n_blocks = xf.shape[-2] // block_size
    blocked = xf.reshape(*lead, n_blocks, block_size, xf.shape[-1])
    mn = blocked.min(axis=-2, keepdims=True)
    mx = blocked.max(axis=-2, keepdims=True)
    scale = np.maximum((mx - mn) / F32(255.0), SCALE_FLOOR).astype(F32)
    zp = np.clip(np.rint(-mn / scale), F32(0), F32(255)).astype(F32)
    qu = np.clip(np.rint(blocked / scale + zp), F32(0), F32(255))
    values = (qu.astype(np.int16) - 128).astype(np.int8)
    return OracleQuant(values, scale, zp.astype(np.int16), block_size, original_shape)


def dequantize(q: OracleQuant) -> np.ndarray:
    """Dequantize either KV format: int8 values are the affine INT8 format above, uint8 values
    the FP8 E4M3 codes of oracle/fp8.py."""

    if q.values.dtype == np.uint8:
        from .fp8 import dequantize_fp8_per_block

        return dequantize_fp8_per_block(q)
    return dequantize_int8_per_block(q)


def estimate_quantized_bytes(q: OracleQuant) -> int:
    """values + 4 B per scale + 2 B per zero point (quant.py:232-247)."""

    return int(q.values.size + q.scale.size * 4 + q.zero_point.size * 2)


def quantize_int8_symmetric_per_token(x: np.ndarray) -> OracleQuant:
    """Symmetric absmax INT8, one fp32 scale per token row (per head): a KV format offered
    beside the reference's.  Not a reference function (the reference quantizer is the affine
    per-block one above); pinned by closed forms and a brute-force nearest-code check in
    tests/test_oracle.py.

        scale = max(absmax(row) / 127, 1e-8)      (float32 division)
        q     = clamp(rint(x / scale), -127, 127) (float32 division, half-even)

    Expressed in the affine layout with block_size 1 and zero point 128, so that
    dequantize_int8_per_block gives q * scale and every affine consumer reads it unchanged.
    """

    if x.ndim < 2:
        raise ValueError("x needs sequence and feature axes")
    if x.shape[-1] <= 0 or x.shape[-2] <= 0:
        raise ValueError("sequence and feature axes must be non-empty")
    original_shape = tuple(int(s) for s in x.shape)
    xf = np.asarray(x, dtype=F32)
    am = np.abs(xf).max(axis=-1, keepdims=True)
    scale = np.maximum(am / F32(127.0), SCALE_FLOOR).astype(F32)
    q = np.clip(np.rint(xf / scale), F32(-127), F32(127)).astype(np.int8)
    lead = xf.shape[:-2]
    S, D = xf.shape[-2], xf.shape[-1]
    values = q.reshape(*lead, S, 1, D)
    zero = np.full((*lead, S, 1, 1), 128, dtype=np.int16)
    return OracleQuant(values, scale.reshape(*lead, S, 1, 1), zero, 1, original_shape)
