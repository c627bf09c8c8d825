"""Write the golden fixtures in this directory from the reference implementation.

Run once, in a container where the reference checkout exists:

    python tests/golden/make_golden.py /root/reference

It imports the reference package (pure Python + torch CPU) and records
input/output vectors for the functions whose exact bits no closed form pins:

* ``PagedKVCache.append``          whole-store requantization (paged.py:463-557)
* ``PagedKVAllocator`` lifecycle  page reuse and stale-row requant (paged.py:17-255)
* ``quantize_int8_per_block``     tail padding, constant and zero blocks (quant.py:94-165)
* ``PagedKVCache.from_dense``      shuffled/interleaved tables (paged.py:302-419)

The fixtures are data only (``.npz``, no pickles).  Nothing at test time reads
the reference checkout.
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent


def _np(t: torch.Tensor) -> np.ndarray:
    # copy: a CPU tensor's .numpy() shares memory, and the allocator store is mutated in place
    return t.detach().cpu().numpy().copy()


def _quant_fields(prefix: str, q) -> dict:
    return {
        f"{prefix}_values": _np(q.values),
        f"{prefix}_scale": _np(q.scale),
        f"{prefix}_zero": _np(q.zero_point),
        f"{prefix}_shape": np.asarray(q.original_shape, dtype=np.int64),
        f"{prefix}_block": np.asarray(q.block_size, dtype=np.int64),
    }


def _cache_fields(prefix: str, cache) -> dict:
    out = {}
    out.update(_quant_fields(f"{prefix}_k", cache.k_quant))
    out.update(_quant_fields(f"{prefix}_v", cache.v_quant))
    out[f"{prefix}_table"] = _np(cache.block_table)
    out[f"{prefix}_lengths"] = _np(cache.lengths)
    out[f"{prefix}_max_seq_len"] = np.asarray(cache.max_seq_len, dtype=np.int64)
    return out


def make_quant(fs) -> dict:
    g = torch.Generator().manual_seed(1234)
    data = {}
    cases = {
        "ragged_f32": (torch.randn(2, 3, 19, 16, generator=g), 8),
        "f16_block16": (torch.randn(2, 2, 37, 64, generator=g).to(torch.float16), 16),
        "scaled_f32": (torch.randn(1, 2, 32, 128, generator=g) * 7.5 + 1.25, 16),
        "positive_f32": (torch.rand(1, 1, 16, 32, generator=g) + 0.5, 16),
    }
    const = torch.zeros(1, 2, 16, 8)
    const[0, 1] = 3.0
    cases["const_zero"] = (const, 16)
    for name, (x, bs) in cases.items():
        q = fs.quantize_int8_per_block(x, block_size=bs)
        data[f"{name}_x"] = _np(x)
        data.update(_quant_fields(name, q))
        data[f"{name}_deq"] = _np(fs.dequantize_int8_per_block(q))
    data["names"] = np.asarray(list(cases))
    return data


def make_layouts(fs) -> dict:
    g = torch.Generator().manual_seed(99)
    data = {}
    k = torch.randn(3, 2, 17, 8, generator=g)
    v = torch.randn(3, 2, 17, 8, generator=g)
    data["k"], data["v"] = _np(k), _np(v)
    lengths = torch.tensor([17, 11, 5], dtype=torch.int64)
    data["lengths"] = _np(lengths)
    for layout, seed in (("contiguous", 0), ("shuffled", 13), ("shuffled", 0), ("interleaved", 0)):
        cache = fs.PagedKVCache.from_dense(k, v, block_size=4, lengths=lengths,
                                           block_table_pattern=layout, layout_seed=seed)
        data.update(_cache_fields(f"{layout}{seed}", cache))
    # Shuffled tables at benchmark-like sizes (torch CPU randperm, seeded).
    for batch, n, seed in ((8, 256, 0), (16, 256, 0), (8, 128, 0)):
        gen = torch.Generator().manual_seed(seed)
        data[f"randperm_{batch * n}_{seed}"] = _np(torch.randperm(batch * n, generator=gen))
    return data


def make_append(fs) -> dict:
    g = torch.Generator().manual_seed(4321)
    data = {}
    cases = {
        # name: (B, H, S, D, page, T, lengths or None, layout)
        "ref_test": (2, 2, 5, 8, 4, 3, None, "contiguous"),
        "ref_test2": (2, 2, 7, 8, 4, 2, None, "contiguous"),
        "ragged": (3, 2, 9, 16, 4, 6, [9, 4, 1], "shuffled"),
        "cross_page": (2, 3, 16, 32, 16, 20, [16, 13], "interleaved"),
    }
    for name, (B, H, S, D, page, T, lens, layout) in cases.items():
        k = torch.randn(B, H, S, D, generator=g)
        v = torch.randn(B, H, S, D, generator=g)
        kn = torch.randn(B, H, T, D, generator=g)
        vn = torch.randn(B, H, T, D, generator=g)
        lengths = None if lens is None else torch.tensor(lens, dtype=torch.int64)
        cache = fs.PagedKVCache.from_dense(k, v, block_size=page, lengths=lengths,
                                           block_table_pattern=layout, layout_seed=5)
        out = cache.append(kn, vn)
        data[f"{name}_k"], data[f"{name}_v"] = _np(k), _np(v)
        data[f"{name}_kn"], data[f"{name}_vn"] = _np(kn), _np(vn)
        data.update(_cache_fields(f"{name}_in", cache))
        data.update(_cache_fields(f"{name}_out", out))
        q = torch.randn(B, H, D, generator=g)
        data[f"{name}_q"] = _np(q)
        data[f"{name}_attn"] = _np(fs.paged_quant_attention(q, out))
    data["names"] = np.asarray(list(cases))
    return data


def make_allocator(fs) -> dict:
    """Replays a fixed lifecycle script and records the store after every op."""

    g = torch.Generator().manual_seed(777)
    H, D, bs, cap = 2, 8, 4, 8
    alloc = fs.PagedKVAllocator(capacity_blocks=cap, heads=H, head_dim=D, block_size=bs)
    script = [
        ("add", 10, 5), ("add", 20, 3), ("append", 10, 4), ("add", 30, 7),
        ("release", 20, 0), ("add", 40, 1), ("append", 40, 6), ("append", 30, 1),
        ("release", 10, 0), ("add", 50, 9), ("append", 50, 3),
    ]
    data = {"script": np.asarray([(0 if op == "add" else 1 if op == "append" else 2, rid, n)
                                  for op, rid, n in script], dtype=np.int64)}
    for step, (op, rid, n) in enumerate(script):
        if op == "add":
            k = torch.randn(1, H, n, D, generator=g)
            v = torch.randn(1, H, n, D, generator=g)
            data[f"s{step}_k"], data[f"s{step}_v"] = _np(k), _np(v)
            alloc.add_request(rid, k, v)
        elif op == "append":
            k = torch.randn(1, H, n, D, generator=g)
            v = torch.randn(1, H, n, D, generator=g)
            data[f"s{step}_k"], data[f"s{step}_v"] = _np(k), _np(v)
            alloc.append_request(rid, k, v)
        else:
            alloc.release_request(rid)
        data[f"s{step}_kvalues"] = _np(alloc.k_quant.values)
        data[f"s{step}_kscale"] = _np(alloc.k_quant.scale)
        data[f"s{step}_kzero"] = _np(alloc.k_quant.zero_point)
        data[f"s{step}_vvalues"] = _np(alloc.v_quant.values)
        data[f"s{step}_vscale"] = _np(alloc.v_quant.scale)
        data[f"s{step}_vzero"] = _np(alloc.v_quant.zero_point)
        live = alloc.live_request_ids
        data[f"s{step}_live"] = np.asarray(live, dtype=np.int64)
        if live:
            cache = alloc.to_cache(live)
            data[f"s{step}_table"] = _np(cache.block_table)
            data[f"s{step}_lengths"] = _np(cache.lengths)
        data[f"s{step}_allocated"] = np.asarray(alloc.stats()["allocated_blocks"])
    data["config"] = np.asarray([H, D, bs, cap], dtype=np.int64)
    return data


def main() -> None:
    ref = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
    sys.path.insert(0, str(ref / "src"))
    import flashspec as fs  # the reference package

    torch.set_num_threads(1)
    np.savez_compressed(HERE / "quant_golden.npz", **make_quant(fs))
    np.savez_compressed(HERE / "layout_golden.npz", **make_layouts(fs))
    np.savez_compressed(HERE / "append_golden.npz", **make_append(fs))
    np.savez_compressed(HERE / "allocator_golden.npz", **make_allocator(fs))
    for p in sorted(HERE.glob("*.npz")):
        print(p.name, p.stat().st_size)


if __name__ == "__main__":
    main()
