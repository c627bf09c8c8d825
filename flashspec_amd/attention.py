"""Portable decode-attention paths (reference src/flashspec/attention.py).

These are the reference's own PyTorch paths — dequantize to dense float32, then
attend — kept because they are public API and because ``*_triton`` entry points
route CPU tensors to them (the reference's fallback contract).  They materialize
dense K/V; the HIP kernels in ``triton_fused`` / ``triton_paged`` do not.
"""

from __future__ import annotations

import math
from typing import Dict, Optional, Tuple

import torch

from .paged import PagedKVCache
from .quant import QuantizedTensor, build_compression_stats, dequantize_int8_per_block, estimate_quantized_bytes


def _validate_decode_shapes(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> None:
    """attention.py:17-42."""

    if q.ndim != 3:
        raise ValueError("q must be [batch, heads, head_dim]")
    if k.ndim != 4 or v.ndim != 4:
        raise ValueError("k and v must be [batch, heads, seq_len, head_dim]")
    if k.shape != v.shape:
        raise ValueError("k and v must have the same shape")
    if q.shape[0] != k.shape[0] or q.shape[1] != k.shape[1] or q.shape[2] != k.shape[3]:
        raise ValueError("q batch, heads and head_dim must match k/v")


def _sequence_mask(seq_len: int, lengths: Optional[torch.Tensor], device: torch.device) -> Optional[torch.Tensor]:
    """[batch, seq_len] mask, True past each row's length (attention.py:45-67)."""

    if lengths is None:
        return None
    positions = torch.arange(seq_len, device=device).unsqueeze(0)
    return positions >= lengths.to(device).unsqueeze(1)


def reference_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                        lengths: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Single-query decode attention in float32 (attention.py:70-121).

    Masked positions get float32 min, so a zero-length row averages V uniformly.
    """

    _validate_decode_shapes(q, k, v)
    scale = 1.0 / math.sqrt(q.shape[-1])
    scores = torch.einsum("bhd,bhsd->bhs", q.to(torch.float32), k.to(torch.float32)) * scale
    mask = _sequence_mask(k.shape[-2], lengths, k.device)
    if mask is not None:
        scores = scores.masked_fill(mask[:, None, :], torch.finfo(scores.dtype).min)
    probs = torch.softmax(scores, dim=-1)
    return torch.einsum("bhs,bhsd->bhd", probs, v.to(torch.float32)).to(q.dtype)


def fused_dequant_attention(q: torch.Tensor, k_quant: QuantizedTensor, v_quant: QuantizedTensor,
                            lengths: Optional[torch.Tensor] = None, return_stats: bool = False,
                            ) -> torch.Tensor | Tuple[torch.Tensor, Dict[str, float]]:
    """Kernel-1 API, portable path: dequantize K/V then ``reference_attention`` (attention.py:124-168)."""

    k = dequantize_int8_per_block(k_quant, dtype=torch.float32)
    v = dequantize_int8_per_block(v_quant, dtype=torch.float32)
    out = reference_attention(q, k, v, lengths=lengths)
    if not return_stats:
        return out
    dense_bytes = 2 * k.numel() * q.element_size()
    quant_bytes = estimate_quantized_bytes(k_quant) + estimate_quantized_bytes(v_quant)
    return out, build_compression_stats(dense_bytes, quant_bytes, materializes_dense_kv=True)


def paged_quant_attention(q: torch.Tensor, cache: PagedKVCache, return_stats: bool = False,
                          ) -> torch.Tensor | Tuple[torch.Tensor, Dict[str, float]]:
    """Kernel-2 API, portable path: ``cache.to_dense()`` then attend with ``cache.lengths`` (attention.py:171-223)."""

    k, v = cache.to_dense()
    out = reference_attention(q, k, v, lengths=cache.lengths)
    if not return_stats:
        return out
    dense_bytes = 2 * k.numel() * q.element_size()
    stats = build_compression_stats(
        dense_bytes, cache.estimated_bytes(), materializes_dense_kv=True,
        physical_blocks=float(cache.block_table.ge(0).sum().item()),
    )
    return out, stats
