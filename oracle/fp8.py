"""Oracle: FP8 (OCP E4M3, "e4m3fn") per-block KV quantization — TEST INFRASTRUCTURE ONLY.

A KV format offered beside the reference's INT8 ones (the reference lists FP8 among the
formats to compare, doc/TODO.MD:241-255, without implementing it), so this module defines it:

* code format: OCP FP8 E4M3 (1 sign, 4 exponent bits with bias 7, 3 mantissa bits; no
  infinities; S.1111.111 is NaN; largest finite 448; subnormals m * 2^-9);
* per block of ``block_size`` tokens x head_dim (zero-padded like the INT8 quantizer, the
  padding taking part in the maximum), one float32 scale and no zero point:

      scale = max(absmax(block) / 448, 1e-8)        (float32 division)
      code  = E4M3_RNE(clamp(x / scale, -448, 448)) (float32 division, nearest-even)
      x'    = float32(code) * scale                 (one float32 product)

  Stored in the INT8 affine layout's shapes (values [..., nb, block, D] as raw codes, scale
  and an all-zero zero point [..., nb, 1, 1]), so the paged and fused stores keep one layout.

The encoder here works from the value table of the format, not from any library; the tests
(tests/test_oracle.py) pin it against torch's CPU float8_e4m3fn conversion on every code,
every rounding tie and random values, and pin the block quantizer by closed forms (the block
maximum maps to the extreme code, a zero block to scale 1e-8 and code 0, the error bound of a
3-bit mantissa) and a brute-force nearest-code check.  NaN inputs are not part of the format.
"""

from __future__ import annotations

import numpy as np

from .quant import F32, SCALE_FLOOR, OracleQuant, pad_sequence_dim

E4M3_MAX = 448.0
E4M3_NAN_CODES = (0x7F, 0xFF)


def e4m3_table() -> np.ndarray:
    """float64 value of each of the 256 codes (NaN for the two NaN codes)."""

    out = np.empty(256, dtype=np.float64)
    for c in range(256):
        sign = -1.0 if c & 0x80 else 1.0
        e = (c >> 3) & 0xF
        m = c & 0x7
        if e == 0xF and m == 0x7:
            out[c] = np.nan
        elif e == 0:
            out[c] = sign * m * 2.0 ** -9
        else:
            out[c] = sign * (1.0 + m / 8.0) * 2.0 ** (e - 7)
    return out


_TABLE = e4m3_table()
_POS = _TABLE[:0x7F]  # codes 0x00..0x7E: 0 .. 448, strictly increasing


def decode_e4m3(codes: np.ndarray) -> np.ndarray:
    """Codes (uint8) to float32 values (exact)."""

    return _TABLE[np.asarray(codes, dtype=np.uint8)].astype(F32)


def encode_e4m3_rne(x: np.ndarray) -> np.ndarray:
    """Round float32 values with |x| <= 448 to the nearest E4M3 code, ties to the even code."""

    x = np.asarray(x, dtype=F32)
    if np.isnan(x).any() or (np.abs(x) > E4M3_MAX).any():
        raise ValueError("encode_e4m3_rne takes finite values with |x| <= 448 (clamp first)")
    a = np.abs(x.astype(np.float64))
    hi = np.clip(np.searchsorted(_POS, a, side="left"), 0, len(_POS) - 1)
    lo = np.clip(hi - 1, 0, len(_POS) - 1)
    d_lo = a - _POS[lo]
    d_hi = _POS[hi] - a
    pick_hi = (d_hi < d_lo) | ((d_hi == d_lo) & (hi % 2 == 0))
    code = np.where(pick_hi, hi, lo).astype(np.uint8)
    code = np.where(_POS[code] == a, code, code)  # exact hits: searchsorted(left) lands on them
    return (code | np.where(np.signbit(x), 0x80, 0).astype(np.uint8)).astype(np.uint8)


def quantize_fp8_per_block(x: np.ndarray, block_size: int = 16) -> OracleQuant:
    """FP8 E4M3 with one float32 scale per [block_size, head_dim] block (module docstring)."""

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
    amax = np.abs(blocked).max(axis=(-2, -1), keepdims=True)
    scale = np.maximum(amax / F32(E4M3_MAX), SCALE_FLOOR).astype(F32)
    y = np.clip((blocked / scale).astype(F32), F32(-E4M3_MAX), F32(E4M3_MAX))
    codes = encode_e4m3_rne(y)
    zero = np.zeros(scale.shape, dtype=np.int16)
    return OracleQuant(codes, scale, zero, block_size, original_shape)


def dequantize_fp8_per_block(q: OracleQuant) -> np.ndarray:
    """``float32(code) * scale``, then crop the padding."""

    x = (decode_e4m3(q.values) * q.scale.astype(F32)).astype(F32)
    lead = q.original_shape[:-2]
    seq_len, head_dim = q.original_shape[-2], q.original_shape[-1]
    return x.reshape(*lead, -1, head_dim)[..., :seq_len, :].astype(F32)
