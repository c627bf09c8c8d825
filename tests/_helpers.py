"""Shared test helpers: conversions between oracle (numpy) and package (torch) objects."""

from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

import flashspec_amd as fa
from oracle import attention as oa
from oracle import paged as op
from oracle import quant as oq

GOLDEN = Path(__file__).resolve().parent / "golden"

# Output tolerance for attention in fp16 (north star): max-abs 2e-3, and max-rel 1e-2
# wherever |reference| >= 1e-2.  The reference output is cast to the q dtype first,
# as the reference path does (attention.py:121).
ATOL = 2.0e-3
RTOL = 1.0e-2
REL_FLOOR = 1.0e-2


def randn(shape, seed: int, dtype=torch.float16) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    return torch.randn(shape, generator=g, dtype=torch.float32).to(dtype)


def np_of(t: torch.Tensor) -> np.ndarray:
    """numpy copy; bf16 as float32, FP8 E4M3 codes as uint8 (the oracle's FP8 values)."""

    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        t = t.to(torch.float32)
    if t.dtype == torch.float8_e4m3fn:
        t = t.view(torch.uint8)
    return t.numpy()


def to_qt(q: oq.OracleQuant, device) -> fa.QuantizedTensor:
    values = torch.from_numpy(np.ascontiguousarray(q.values))
    if values.dtype == torch.uint8:  # the oracle's FP8 codes
        values = values.view(torch.float8_e4m3fn)
    return fa.QuantizedTensor(
        values.to(device),
        torch.from_numpy(np.ascontiguousarray(q.scale)).to(device),
        torch.from_numpy(np.ascontiguousarray(q.zero_point)).to(device),
        int(q.block_size), tuple(int(s) for s in q.original_shape),
    )


def from_qt(q: fa.QuantizedTensor) -> oq.OracleQuant:
    return oq.OracleQuant(np_of(q.values), np_of(q.scale), np_of(q.zero_point), int(q.block_size),
                          tuple(int(s) for s in q.original_shape))


def to_cache(c: op.OracleCache, device) -> fa.PagedKVCache:
    return fa.PagedKVCache(to_qt(c.k_quant, device), to_qt(c.v_quant, device),
                           torch.from_numpy(c.block_table.astype(np.int64)).to(device),
                           torch.from_numpy(c.lengths.astype(np.int64)).to(device), int(c.block_size),
                           int(c.max_seq_len))


def from_cache(c: fa.PagedKVCache) -> op.OracleCache:
    return op.OracleCache(from_qt(c.k_quant), from_qt(c.v_quant), np_of(c.block_table).astype(np.int64),
                          np_of(c.lengths).astype(np.int64), int(c.block_size), int(c.max_seq_len))


def assert_quant_equal(a, b, what: str = "") -> None:
    """Bit-exact equality of values, scale and zero point."""

    av, bv = np.asarray(a.values), np.asarray(b.values)
    assert av.shape == bv.shape, (what, av.shape, bv.shape)
    assert np.array_equal(av, bv), f"{what}: int8 values differ at {np.argwhere(av != bv)[:5].tolist()}"
    assert np.array_equal(np.asarray(a.scale, np.float32).view(np.uint32).ravel(),
                          np.asarray(b.scale, np.float32).view(np.uint32).ravel()), f"{what}: scale bits differ"
    assert np.array_equal(np.asarray(a.zero_point).ravel(), np.asarray(b.zero_point).ravel()), f"{what}: zero differs"


def cast_like_q(ref: np.ndarray, q_dtype: torch.dtype) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(ref, dtype=np.float32)).to(q_dtype).to(torch.float32).numpy()


def attention_errors(actual: torch.Tensor, ref: np.ndarray, q_dtype: torch.dtype):
    a = np_of(actual.to(torch.float32)).astype(np.float64)
    r = cast_like_q(ref, q_dtype).astype(np.float64)
    diff = np.abs(a - r)
    big = np.abs(r) >= REL_FLOOR
    max_rel = float((diff[big] / np.abs(r[big])).max()) if big.any() else 0.0
    return float(diff.max()) if diff.size else 0.0, max_rel


def assert_attention_close(actual: torch.Tensor, ref: np.ndarray, q_dtype: torch.dtype, what: str = "") -> None:
    assert tuple(actual.shape) == tuple(ref.shape), (what, actual.shape, ref.shape)
    assert actual.dtype == q_dtype
    assert torch.isfinite(actual.to(torch.float32)).all(), f"{what}: non-finite output"
    max_abs, max_rel = attention_errors(actual, ref, q_dtype)
    assert max_abs <= ATOL and max_rel <= RTOL, f"{what}: max_abs={max_abs:.3e} max_rel={max_rel:.3e}"


def oracle_paged_attention(q: torch.Tensor, cache: fa.PagedKVCache) -> np.ndarray:
    return oa.paged_quant_attention(np_of(q), from_cache(cache))


def oracle_fused_attention(q: torch.Tensor, kq: fa.QuantizedTensor, vq: fa.QuantizedTensor, lengths=None):
    lens = None if lengths is None else np_of(lengths).astype(np.int64)
    return oa.fused_dequant_attention(np_of(q), from_qt(kq), from_qt(vq), lens)


def load_npz(name: str):
    return np.load(GOLDEN / name, allow_pickle=False)


def golden_quant(d, prefix: str) -> oq.OracleQuant:
    return oq.OracleQuant(d[f"{prefix}_values"], d[f"{prefix}_scale"], d[f"{prefix}_zero"],
                          int(d[f"{prefix}_block"]), tuple(int(s) for s in d[f"{prefix}_shape"]))


def golden_cache(d, prefix: str) -> op.OracleCache:
    return op.OracleCache(golden_quant(d, f"{prefix}_k"), golden_quant(d, f"{prefix}_v"), d[f"{prefix}_table"],
                          d[f"{prefix}_lengths"], int(d[f"{prefix}_k_block"]), int(d[f"{prefix}_max_seq_len"]))
