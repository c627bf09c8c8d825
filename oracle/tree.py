"""Tree-verification oracle — TEST INFRASTRUCTURE ONLY (imported by tests/ and nowhere else).

Speculative-decoding tree verification over a paged INT8 prefix.  The reference plans this
kernel (reference doc/TODO.MD:186-237: tree mask instead of a causal mask, each node sees the
prefix and its own root path, siblings and other branches masked, a single path reduces to
the paged decode) but does not implement it, so this module defines the semantics:

* request b has N draft nodes in topological order; ``parents[b, n]`` is the parent of node
  n, in [-1, n) (-1: the node hangs off the last committed token);
* node n attends to the prefix tokens [0, lengths[b]) of the paged cache (dequantized as
  ``paged.to_dense`` does) and to the draft tokens on its root path (n and its ancestors),
  whose K/V are unquantized;
* attention math is reference_attention's (scores in float32 scaled by 1/sqrt(D), masked
  entries at finfo(float32).min, softmax, probability-weighted V).

``tree_verify_attention`` builds the explicit dense tree mask; ``tree_verify_f64_loops``
walks the parent pointers per node in float64.  tests/test_oracle.py pins both against each
other and against ``reference_attention`` on explicitly concatenated K/V (chain and star
trees), and checks that malformed trees are rejected.
"""

from __future__ import annotations

import numpy as np

from . import paged as op

F32 = np.float32


def validate_parents(parents: np.ndarray) -> np.ndarray:
    """Reject anything but a forest in topological order: every parent in [-1, own index)."""

    p = np.asarray(parents)
    if p.ndim != 2:
        raise ValueError("parents must be [batch, nodes]")
    idx = np.arange(p.shape[1])[None, :]
    if (p < -1).any() or (p >= idx).any():
        raise ValueError("parents[b, n] must lie in [-1, n): cycles, forward edges and orphans are invalid")
    return p.astype(np.int64)


def path_mask(parents: np.ndarray) -> np.ndarray:
    """mask[b, n, j] = draft node j lies on node n's root path (n itself included)."""

    p = validate_parents(parents)
    B, N = p.shape
    mask = np.zeros((B, N, N), dtype=bool)
    for b in range(B):
        for n in range(N):
            mask[b, n, n] = True
            if p[b, n] >= 0:
                mask[b, n] |= mask[b, p[b, n]]
    return mask


def tree_verify_attention(q, cache: op.OracleCache, draft_k, draft_v, parents) -> np.ndarray:
    """Dense tree-mask formulation.  q, draft_k, draft_v: [B, N, H, D]; returns [B, N, H, D] float32."""

    q = np.asarray(q, dtype=F32)
    dk = np.asarray(draft_k, dtype=F32)
    dv = np.asarray(draft_v, dtype=F32)
    B, N, H, D = q.shape
    kp, vp = op.to_dense(cache)  # [B, H, S, D]
    S = kp.shape[2]
    keys = np.concatenate([kp, dk.transpose(0, 2, 1, 3)], axis=2)  # [B, H, S + N, D]
    vals = np.concatenate([vp, dv.transpose(0, 2, 1, 3)], axis=2)
    allowed = np.zeros((B, N, S + N), dtype=bool)
    allowed[:, :, :S] = np.arange(S)[None, None, :] < np.asarray(cache.lengths)[:, None, None]
    allowed[:, :, S:] = path_mask(parents)
    scale = F32(1.0 / np.sqrt(D))
    scores = np.einsum("bnhd,bhkd->bhnk", q, keys).astype(F32) * scale
    scores = np.where(allowed[:, None, :, :], scores, np.finfo(F32).min)
    scores = scores - scores.max(axis=-1, keepdims=True)
    p = np.exp(scores)
    p = p / p.sum(axis=-1, keepdims=True)
    out = np.einsum("bhnk,bhkd->bnhd", p, vals)
    return out.astype(F32)


def tree_verify_f64_loops(q, cache: op.OracleCache, draft_k, draft_v, parents) -> np.ndarray:
    """Per-node brute force in float64, walking the parent pointers explicitly."""

    q = np.asarray(q, dtype=np.float64)
    dk = np.asarray(draft_k, dtype=np.float64)
    dv = np.asarray(draft_v, dtype=np.float64)
    p = validate_parents(parents)
    B, N, H, D = q.shape
    kp, vp = op.to_dense(cache)
    out = np.zeros((B, N, H, D), dtype=np.float64)
    for b in range(B):
        L = int(cache.lengths[b])
        for n in range(N):
            path = []
            a = n
            while a >= 0:
                path.append(a)
                a = int(p[b, a])
            for h in range(H):
                ks = [kp[b, h, t].astype(np.float64) for t in range(L)] + [dk[b, a, h] for a in path]
                vs = [vp[b, h, t].astype(np.float64) for t in range(L)] + [dv[b, a, h] for a in path]
                s = np.array([q[b, n, h] @ k for k in ks]) / np.sqrt(D)
                w = np.exp(s - s.max())
                w /= w.sum()
                out[b, n, h] = sum(wi * v for wi, v in zip(w, vs))
    return out
