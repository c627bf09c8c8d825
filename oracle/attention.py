"""Oracle: single-query decode attention (test infrastructure only).

Restates reference src/flashspec/attention.py:70-223 in numpy float32.  The
result is returned in float32 *before* the reference's final ``.to(q.dtype)``
cast (attention.py:121); tests compare against it with an explicit tolerance.
"""

from __future__ import annotations

import math
from typing import Optional

import numpy as np

from . import quant as oq

F32 = np.float32
F32_MIN = np.finfo(np.float32).min


def validate_decode_shapes(q: np.ndarray, k: np.ndarray, v: np.ndarray) -> None:
    """Shape rules of attention.py:17-42."""

    if q.ndim != 3:
        raise ValueError("q must be [batch, heads, head_dim]")
    if k.ndim != 4 or v.ndim != 4:
        raise ValueError("k and v must be [batch, heads, seq_len, head_dim]")
    if k.shape != v.shape:
        raise ValueError("k and v must have the same shape")
    if q.shape[0] != k.shape[0] or q.shape[1] != k.shape[1] or q.shape[2] != k.shape[3]:
        raise ValueError("q batch/heads/head_dim must match k/v")


def reference_attention(
    q: np.ndarray, k: np.ndarray, v: np.ndarray, lengths: Optional[np.ndarray] = None
) -> np.ndarray:
    """Dense decode attention (attention.py:70-121).

    ``scores = (q . k) * 1/sqrt(D)`` in float32; positions ``>= lengths[b]`` are
    set to float32 min (so a zero-length row averages V uniformly, as the
    reference does); softmax over the sequence; ``probs . v``.
    """

    validate_decode_shapes(q, k, v)
    q32, k32, v32 = (np.asarray(t, dtype=F32) for t in (q, k, v))
    scale = F32(1.0 / math.sqrt(q.shape[-1]))
    scores = np.einsum("bhd,bhsd->bhs", q32, k32).astype(F32) * scale
    if lengths is not None:
        pos = np.arange(k.shape[-2])[None, :]
        mask = pos >= np.asarray(lengths).reshape(-1, 1)
        scores = np.where(mask[:, None, :], F32_MIN, scores)
    scores = scores - scores.max(axis=-1, keepdims=True)
    e = np.exp(scores, dtype=F32)
    probs = (e / e.sum(axis=-1, keepdims=True)).astype(F32)
    return np.einsum("bhs,bhsd->bhd", probs, v32).astype(F32)


def reference_attention_f64_loops(q, k, v, lengths=None) -> np.ndarray:
    """Float64 brute force with explicit loops — the pin for ``reference_attention``.

    Small shapes only.  Written independently of the vectorised version so that
    a transposed operand or a dropped scale fails the comparison.
    """

    B, H, S, D = k.shape
    out = np.zeros((B, H, D), dtype=np.float64)
    for b in range(B):
        valid = S if lengths is None else int(lengths[b])
        for h in range(H):
            logits = []
            for s in range(S):
                acc = 0.0
                for d in range(D):
                    acc += float(q[b, h, d]) * float(k[b, h, s, d])
                logits.append(acc / math.sqrt(D) if s < valid else -math.inf)
            if valid <= 0:
                weights = [1.0 / S] * S  # every logit equal -> uniform
            else:
                top = max(logits)
                ex = [math.exp(x - top) if x != -math.inf else 0.0 for x in logits]
                tot = sum(ex)
                weights = [e / tot for e in ex]
            for d in range(D):
                out[b, h, d] = sum(weights[s] * float(v[b, h, s, d]) for s in range(S))
    return out


def fused_dequant_attention(q, k_quant: oq.OracleQuant, v_quant: oq.OracleQuant, lengths=None) -> np.ndarray:
    """Oracle for the contiguous INT8 kernel (attention.py:124-168): dequantize, then attend."""

    k = oq.dequantize(k_quant)
    v = oq.dequantize(v_quant)
    return reference_attention(q, k, v, lengths)


def paged_quant_attention(q, cache) -> np.ndarray:
    """Oracle for the paged INT8 kernel (attention.py:171-223): ``to_dense`` then attend."""

    from .paged import to_dense

    k, v = to_dense(cache)
    return reference_attention(q, k, v, cache.lengths)
