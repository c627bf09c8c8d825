"""Serving decode loop on the paged allocator (reference src/flashspec/serving.py, benchmarks/e2e_serving.py).

``run_decode_simulation(ServingConfig)`` keeps the reference's request lifecycle,
random-input draw order, timing points and result keys, with one change the
reference's own design calls for: attention goes through
``paged_quant_attention_triton`` (the HIP kernel on GPU, the portable path on CPU)
instead of the portable path only (serving.py:118,139 call ``paged_quant_attention``).
The allocator's prompt writes and per-step appends run as batched HIP page-update
launches on GPU.

``build_request_pool`` and ``decode_step`` are the serving-at-scale pieces: a
fragmented page pool of ragged requests, and one decode step that appends one token
per request and then attends over the updated cache.

    python -m flashspec_amd.serving --requests 8 --prompt-lens 512,2048 --decode-steps 16 --json
"""

from __future__ import annotations

import argparse
import json
from dataclasses import dataclass
from time import perf_counter
from typing import Dict, Sequence

import torch

from .paged import PagedKVAllocator
from .runtime import device_name, resolve_device, resolve_dtype, synchronize
from .triton_paged import paged_quant_attention_triton

DTYPE_CHOICES = ["auto", "float16", "fp16", "bfloat16", "bf16", "float32", "fp32"]


@dataclass(frozen=True)
class ServingConfig:
    """Decode-simulation settings (serving.py:14-30)."""

    requests: int = 8
    prompt_len: int = 128
    prompt_lens: tuple[int, ...] | None = None
    prompt_length_distribution: str = "uniform"
    decode_steps: int = 16
    request_life_steps: int = 0
    heads: int = 8
    head_dim: int = 64
    block_size: int = 16
    allocator_blocks: int | None = None
    seed: int = 0
    device: str = "auto"
    dtype: str = "auto"


def _validate_config(config: ServingConfig) -> None:
    if config.requests <= 0:
        raise ValueError("requests must be positive")
    if config.prompt_len <= 0:
        raise ValueError("prompt_len must be positive")
    if config.decode_steps < 0:
        raise ValueError("decode_steps must be >= 0")
    if config.request_life_steps < 0:
        raise ValueError("request_life_steps must be >= 0")
    if config.heads <= 0 or config.head_dim <= 0:
        raise ValueError("heads and head_dim must be positive")
    if config.block_size <= 0:
        raise ValueError("block_size must be positive")


def _resolve_prompt_lens(config: ServingConfig) -> tuple[int, ...]:
    lens = config.prompt_lens if config.prompt_lens is not None else (config.prompt_len,)
    if not lens:
        raise ValueError("prompt_lens must not be empty")
    if any(length <= 0 for length in lens):
        raise ValueError("prompt_lens must all be positive")
    return tuple(int(length) for length in lens)


def _estimate_allocator_blocks(config: ServingConfig, prompt_lens: Sequence[int]) -> int:
    """Enough pages for every live request's longest prompt plus its decode tokens (serving.py:217-227)."""

    if config.allocator_blocks is not None:
        if config.allocator_blocks <= 0:
            raise ValueError("allocator_blocks must be positive")
        return int(config.allocator_blocks)
    tokens = max(prompt_lens) + max(1, config.decode_steps)
    return max(1, config.requests * ((tokens + config.block_size - 1) // config.block_size))


def _sample_prompt_len(prompt_lens: Sequence[int], *, distribution: str, request_index: int,
                       generator: torch.Generator, device: torch.device) -> int:
    """cycle/uniform, random (one seeded draw), or bimodal first/last (serving.py:230-247)."""

    mode = distribution.strip().lower()
    if mode in {"uniform", "cycle"}:
        return int(prompt_lens[request_index % len(prompt_lens)])
    if mode == "random":
        idx = int(torch.randint(len(prompt_lens), (1,), generator=generator, device=device).item())
        return int(prompt_lens[idx])
    if mode == "bimodal":
        if len(prompt_lens) == 1:
            return int(prompt_lens[0])
        return int(prompt_lens[0] if request_index % 2 == 0 else prompt_lens[-1])
    raise ValueError("prompt_length_distribution must be uniform, random or bimodal")


def _random_kv(*, batch: int, heads: int, tokens: int, head_dim: int, generator: torch.Generator,
               device: torch.device, dtype: torch.dtype) -> tuple[torch.Tensor, torch.Tensor]:
    shape = (batch, heads, tokens, head_dim)
    return (torch.randn(shape, generator=generator, device=device, dtype=dtype),
            torch.randn(shape, generator=generator, device=device, dtype=dtype))


def run_decode_simulation(config: ServingConfig) -> Dict[str, float | int | str | list[int]]:
    """Prefill, first attention (TTFT), decode steps with append, optional finish/arrival (serving.py:33-190)."""

    _validate_config(config)
    device = resolve_device(config.device)
    dtype = resolve_dtype(config.dtype, device)
    generator = torch.Generator(device=device)
    generator.manual_seed(config.seed)
    prompt_lens = _resolve_prompt_lens(config)
    allocator = PagedKVAllocator(capacity_blocks=_estimate_allocator_blocks(config, prompt_lens), heads=config.heads,
                                 head_dim=config.head_dim, block_size=config.block_size, device=device, dtype=dtype)
    state = {"next_id": 0, "prefill_ms": 0.0, "arrival_prefill_ms": 0.0, "arrivals": 0}
    active: list[int] = []
    generated: dict[int, int] = {}
    request_prompt_lens: dict[int, int] = {}

    def add_request(*, initial: bool) -> int:
        rid = state["next_id"]
        state["next_id"] += 1
        plen = _sample_prompt_len(prompt_lens, distribution=config.prompt_length_distribution, request_index=rid,
                                  generator=generator, device=device)
        k, v = _random_kv(batch=1, heads=config.heads, tokens=plen, head_dim=config.head_dim, generator=generator,
                          device=device, dtype=dtype)
        synchronize(device)
        t0 = perf_counter()
        allocator.add_request(rid, k, v)
        synchronize(device)
        state["prefill_ms" if initial else "arrival_prefill_ms"] += (perf_counter() - t0) * 1000.0
        state["arrivals"] += 1
        generated[rid] = 0
        request_prompt_lens[rid] = plen
        return rid

    for _ in range(config.requests):
        active.append(add_request(initial=True))

    synchronize(device)
    t0 = perf_counter()
    first_cache = allocator.to_cache(active)
    first_q = torch.randn((len(active), config.heads, config.head_dim), generator=generator, device=device,
                          dtype=dtype)
    _ = paged_quant_attention_triton(first_q, first_cache)
    synchronize(device)
    first_attention_ms = (perf_counter() - t0) * 1000.0

    decode_ms = 0.0
    generated_tokens = 0
    finishes = 0
    for _step in range(config.decode_steps):
        if not active:
            break
        synchronize(device)
        t0 = perf_counter()
        cache = allocator.to_cache(active)
        q = torch.randn((len(active), config.heads, config.head_dim), generator=generator, device=device,
                        dtype=dtype)
        out = paged_quant_attention_triton(q, cache)
        next_k = out.unsqueeze(2).to(dtype=dtype)
        next_v = torch.tanh(out).unsqueeze(2).to(dtype=dtype)
        allocator.append_batch(active, next_k, next_v)
        synchronize(device)
        decode_ms += (perf_counter() - t0) * 1000.0
        for rid in active:
            generated[rid] += 1
        generated_tokens += len(active)
        if config.request_life_steps > 0:
            done = [rid for rid in active if generated[rid] >= config.request_life_steps]
            for rid in done:
                allocator.release_request(rid)
                active.remove(rid)
                generated.pop(rid, None)
                finishes += 1
            for _ in done:
                active.append(add_request(initial=False))

    stats = allocator.stats()
    return {
        "device": str(device), "device_name": device_name(device), "dtype": str(dtype).replace("torch.", ""),
        "requests": config.requests, "prompt_len": config.prompt_len, "prompt_lens": list(prompt_lens),
        "prompt_length_distribution": config.prompt_length_distribution,
        "average_prompt_len": sum(request_prompt_lens.values()) / max(1, len(request_prompt_lens)),
        "decode_steps": config.decode_steps, "request_life_steps": config.request_life_steps,
        "arrivals": state["arrivals"], "finishes": finishes,
        "prefill_ms": state["prefill_ms"], "arrival_prefill_ms": state["arrival_prefill_ms"],
        "total_prefill_ms": state["prefill_ms"] + state["arrival_prefill_ms"],
        "first_attention_ms": first_attention_ms, "decode_ms": decode_ms,
        "ttft_ms": state["prefill_ms"] + first_attention_ms,
        "tpot_ms": decode_ms / max(1, config.decode_steps),
        "tokens_per_second": generated_tokens / max(1.0e-9, decode_ms / 1000.0),
        "generated_tokens": generated_tokens,
        "attention_backend": "hip" if device.type == "cuda" else "portable",
        **stats,
    }


# ---- serving at scale ----------------------------------------------------------------------------

def build_request_pool(lengths: Sequence[int], *, heads: int, head_dim: int, block_size: int = 16,
                       headroom_tokens: int = 16, seed: int = 0, device: torch.device | str = "cuda",
                       dtype: torch.dtype = torch.float16) -> tuple[PagedKVAllocator, list[int]]:
    """A fragmented page pool holding one request per entry of ``lengths``.

    Pool policy (the reference has no single structure for this): capacity covers every
    request plus ``headroom_tokens`` of decode growth, the free list is shuffled with
    ``seed`` so each request's pages are scattered over the pool, and prompt K/V are
    seeded N(0,1) values drawn per request.
    """

    dev = torch.device(device)
    pages = sum((L + headroom_tokens + block_size - 1) // block_size for L in lengths)
    alloc = PagedKVAllocator(capacity_blocks=max(1, pages), heads=heads, head_dim=head_dim, block_size=block_size,
                             device=dev, dtype=dtype)
    alloc.shuffle_free_blocks(seed)
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    rids = []
    for rid, L in enumerate(lengths):
        k, v = _random_kv(batch=1, heads=heads, tokens=int(L), head_dim=head_dim, generator=gen, device=dev,
                          dtype=dtype)
        alloc.add_request(rid, k, v)
        rids.append(rid)
        del k, v
    return alloc, rids


def decode_step(allocator: PagedKVAllocator, request_ids: Sequence[int], q: torch.Tensor, k_new: torch.Tensor,
                v_new: torch.Tensor) -> torch.Tensor:
    """Append one token per request (one batched page-update launch per tensor), then attend.

    ``q`` is ``[n, heads, head_dim]``; ``k_new``/``v_new`` are ``[n, heads, 1, head_dim]``.
    Attention runs over the cache including the appended token.
    """

    allocator.append_batch(request_ids, k_new, v_new)
    return paged_quant_attention_triton(q, allocator.to_cache(request_ids))


def parse_args(argv=None) -> argparse.Namespace:
    p = argparse.ArgumentParser(description="flashspec_amd serving-loop simulation")
    p.add_argument("--requests", type=int, default=8)
    p.add_argument("--prompt-len", type=int, default=128)
    p.add_argument("--prompt-lens", default=None, help="comma-separated prompt length candidates")
    p.add_argument("--prompt-length-distribution", default="uniform", choices=["uniform", "random", "bimodal"])
    p.add_argument("--decode-steps", type=int, default=16)
    p.add_argument("--request-life-steps", type=int, default=0)
    p.add_argument("--heads", type=int, default=8)
    p.add_argument("--head-dim", type=int, default=64)
    p.add_argument("--block-size", type=int, default=16)
    p.add_argument("--allocator-blocks", type=int, default=None)
    p.add_argument("--device", default="auto")
    p.add_argument("--dtype", default="auto", choices=DTYPE_CHOICES)
    p.add_argument("--json", action="store_true")
    return p.parse_args(argv)


def main(argv=None) -> None:
    args = parse_args(argv)
    prompt_lens = None
    if args.prompt_lens:
        prompt_lens = tuple(int(x) for x in args.prompt_lens.split(",") if x.strip())
    result = run_decode_simulation(ServingConfig(
        requests=args.requests, prompt_len=args.prompt_len, prompt_lens=prompt_lens,
        prompt_length_distribution=args.prompt_length_distribution, decode_steps=args.decode_steps,
        request_life_steps=args.request_life_steps, heads=args.heads, head_dim=args.head_dim,
        block_size=args.block_size, allocator_blocks=args.allocator_blocks, device=args.device, dtype=args.dtype))
    if args.json:
        print(json.dumps(result, indent=2))
    else:
        for key, value in result.items():
            print(f"{key}: {value}")


if __name__ == "__main__":
    main()
