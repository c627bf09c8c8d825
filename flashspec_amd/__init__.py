"""flashspec_amd — MI355X (gfx950) INT8 decode-attention hot path of FlashSpec.

Public names match the reference package ``flashspec`` (src/flashspec/__init__.py:1-24),
so its callers can switch by importing this package (or ``flashspec_amd.compat``
to make ``import flashspec`` resolve here).
"""

from .attention import fused_dequant_attention, paged_quant_attention, reference_attention
from .paged import PagedKVAllocator, PagedKVCache
from .quant import (QuantizedTensor, dequantize_fp8_per_block, dequantize_int8_per_block, quantize_fp8_per_block,
                    quantize_int8_per_block, quantize_int8_per_channel, quantize_int8_symmetric_per_token)
from .tree import tree_verify_attention
from .triton_fused import fused_dequant_attention_triton
from .triton_paged import paged_quant_attention_triton

__all__ = [
    "QuantizedTensor",
    "PagedKVCache",
    "PagedKVAllocator",
    "dequantize_fp8_per_block",
    "dequantize_int8_per_block",
    "fused_dequant_attention",
    "fused_dequant_attention_triton",
    "paged_quant_attention",
    "paged_quant_attention_triton",
    "quantize_fp8_per_block",
    "quantize_int8_per_block",
    "quantize_int8_per_channel",
    "quantize_int8_symmetric_per_token",
    "reference_attention",
    "tree_verify_attention",
]
