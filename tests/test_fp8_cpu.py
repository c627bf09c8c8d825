"""FP8 E4M3 KV format on CPU: the portable quantizer bit-exact against the oracle, the
portable attention paths on FP8 stores, and argument checks (flashspec_amd.quant)."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import flashspec_amd as fa
from oracle import attention as oa
from oracle import fp8 as of
from oracle import paged as op
from tests._helpers import assert_quant_equal, from_cache, from_qt


@pytest.mark.parametrize("shape,bs,dtype", [((2, 3, 37, 24), 16, torch.float32), ((1, 2, 64, 128), 32, torch.float16),
                                            ((3, 1, 9, 8), 1, torch.bfloat16)])
def test_portable_fp8_quantize_bit_exact(shape, bs, dtype):
    g = torch.Generator().manual_seed(sum(shape))
    x = (torch.randn(shape, generator=g) * 30).to(dtype)
    got = fa.quantize_fp8_per_block(x, bs)
    ref = of.quantize_fp8_per_block(x.to(torch.float32).numpy(), bs)
    assert_quant_equal(from_qt(got), ref, "portable fp8")
    assert np.array_equal(fa.dequantize_fp8_per_block(got).numpy(), of.dequantize_fp8_per_block(ref))


def test_portable_attention_on_fp8_stores():
    g = torch.Generator().manual_seed(7)
    q = torch.randn((2, 3, 32), generator=g)
    k = torch.randn((2, 3, 50, 32), generator=g)
    v = torch.randn((2, 3, 50, 32), generator=g)
    cache = fa.PagedKVCache.from_dense(k, v, 16, kv_format="fp8_block", block_table_pattern="shuffled")
    got = fa.paged_quant_attention(q, cache)
    ref = oa.paged_quant_attention(q.numpy(), from_cache(cache))
    assert np.abs(got.numpy() - ref).max() < 1e-5
    kq, vq = fa.quantize_fp8_per_block(k, 16), fa.quantize_fp8_per_block(v, 16)
    got_f = fa.fused_dequant_attention(q, kq, vq)
    ref_f = oa.fused_dequant_attention(q.numpy(), from_qt(kq), from_qt(vq))
    assert np.abs(got_f.numpy() - ref_f).max() < 1e-5
    # oracle paged store from the same pages
    ref_cache = op.from_dense(k.numpy(), v.numpy(), 16, kv_format="fp8_block")
    assert ref_cache.k_quant.values.dtype == np.uint8


def test_fp8_argument_checks():
    with pytest.raises(ValueError):
        fa.quantize_fp8_per_block(torch.zeros(4), 16)
    with pytest.raises(ValueError):
        fa.PagedKVCache.from_dense(torch.zeros(1, 1, 4, 8), torch.zeros(1, 1, 4, 8), 4, kv_format="fp4")
    with pytest.raises(ValueError):
        fa.dequantize_fp8_per_block(fa.quantize_int8_per_block(torch.zeros(1, 16, 8), 16))


# ---- per-channel affine INT8 (portable path) ---------------------------------------------------

@pytest.mark.parametrize("shape,bs,dtype", [((2, 3, 45, 24), 16, torch.float32), ((1, 2, 64, 128), 32, torch.float16),
                                            ((2, 1, 10, 8), 4, torch.bfloat16)])
def test_portable_per_channel_bit_exact(shape, bs, dtype):
    from oracle import quant as oq

    g = torch.Generator().manual_seed(sum(shape) + 1)
    x = (torch.randn(shape, generator=g) * torch.rand(shape[-1], generator=g) * 20).to(dtype)
    got = fa.quantize_int8_per_channel(x, bs)
    assert got.scale.shape[-1] == shape[-1]
    assert_quant_equal(from_qt(got), oq.quantize_int8_per_channel(x.to(torch.float32).numpy(), bs), "per-channel")
    cache = fa.PagedKVCache.from_dense(x.to(torch.float32).reshape(1, *x.shape[-3:]) if x.ndim == 3 else
                                       x.to(torch.float32), x.to(torch.float32) if x.ndim == 4 else
                                       x.to(torch.float32).reshape(1, *x.shape[-3:]), bs, kv_format="affine_channel")
    with pytest.raises(ValueError):
        cache.append(torch.zeros(cache.batch_size, cache.num_heads, 1, cache.head_dim),
                     torch.zeros(cache.batch_size, cache.num_heads, 1, cache.head_dim))
