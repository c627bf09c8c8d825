"""Serving decode loop on the paged allocator (reference src/flashspec/serving.py, benchmarks/e2e_serving.py).

``run_decode_simulation(ServingConfig)`` keeps the reference's request lifecycle,
random-input draw order, timing points and result keys, with one change the
reference's own design calls for: attention goes through
``paged_quant_attention_triton`` (the HIP kernel on GPU, the portable path on CPU)
instead of the portable path only (serving.py:118,139 call ``paged_quant_attention``).
On GPU the prompt writes run as batched HIP page-update launches, and the decode loop
keeps the block table and lengths on the device (``DecodeBatch``): per step one attention
launch (``DecodeBatch.attend``) and then one append launch (``DecodeBatch.append``) -- the
reference's order: attend, then append what the attention produced -- with no per-step
table rebuild on the host.

``build_request_pool`` and ``DecodeBatch.step`` are the serving-at-scale pieces: a
fragmented page pool of ragged requests, and a decode step in the other, standard order --
append the step's token (its K/V known beforehand) for every request, then attend over the
updated cache.  ``step`` is one launch, with the append inside the decode kernel, where the
decode grid is one round of workgroups (e.g. 4 requests x 32 heads); larger batches (the
64-request bench workload) take the append launch and then the decode.

    python -m flashspec_amd.serving --requests 8 --prompt-lens 512,2048 --decode-steps 16 --json
"""

from __future__ import annotations

import argparse
import json
import math
from dataclasses import dataclass
from time import perf_counter
from typing import Dict, Sequence

import numpy as np
import torch

from . import _lib
from .paged import PagedKVAllocator, PagedKVCache
from .quant import QuantizedTensor, dequantize_int8_per_block, quantize_int8_per_block
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
    batch: DecodeBatch | None = None  # device-resident table and lengths while the active set is fixed
    for step in range(config.decode_steps):
        if not active:
            break
        synchronize(device)
        t0 = perf_counter()
        if device.type == "cuda" and batch is None:
            horizon = config.decode_steps - step
            if config.request_life_steps > 0:
                horizon = min(horizon, min(config.request_life_steps - generated[r] for r in active))
            batch = DecodeBatch(allocator, active, max_new_tokens=horizon)
        cache = batch.cache() if batch is not None else allocator.to_cache(active)
        q = torch.randn((len(active), config.heads, config.head_dim), generator=generator, device=device,
                        dtype=dtype)
        out = paged_quant_attention_triton(q, cache)
        next_k = out.unsqueeze(2).to(dtype=dtype)
        next_v = torch.tanh(out).unsqueeze(2).to(dtype=dtype)
        if batch is not None:
            batch.append(next_k, next_v)
        else:
            allocator.append_batch(active, next_k, next_v)
        synchronize(device)
        decode_ms += (perf_counter() - t0) * 1000.0
        for rid in active:
            generated[rid] += 1
        generated_tokens += len(active)
        if batch is not None and batch.steps_done == batch.max_new_tokens:
            batch.close()
            batch = None
        if config.request_life_steps > 0:
            done = [rid for rid in active if generated[rid] >= config.request_life_steps]
            if done and batch is not None:
                batch.close()
                batch = None
            for rid in done:
                allocator.release_request(rid)
                active.remove(rid)
                generated.pop(rid, None)
                finishes += 1
            for _ in done:
                active.append(add_request(initial=False))
    if batch is not None:
        batch.close()

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

class DecodeBatch:
    """Device-resident decode state for a fixed set of live requests of a ``PagedKVAllocator``.

    The block table (int32) and the lengths stay on the device between steps.  ``append``
    writes one token per request with a single ``fs_append_tokens_i8`` launch (K and V),
    which reads each request's position from the device lengths and writes the advanced
    lengths to a second buffer, so a decode step needs no host round trip.  ``attend`` runs
    ``paged_quant_attention_triton`` over the current cache.  ``step`` does both in one
    ``fs_paged_decode_append_i8`` launch where the shapes allow it.

    Page policy: pages are taken from the allocator's free list ``reserve_steps`` steps ahead,
    step-major and in request order, the order in which the reference allocator takes them one
    token at a time (paged.py:121-125), so the page ids are the same as step-by-step allocation
    as long as nothing else allocates meanwhile.  ``close`` hands unused reserved pages back to
    the front of the free list in the order they were taken, which restores the allocator's
    state exactly.  While a batch is open, append to its requests only through it.
    On CPU the same bookkeeping drives a portable torch append (dequantize page, replace row,
    requantize), so the host logic is testable without a GPU.
    """

    def __init__(self, allocator: PagedKVAllocator, request_ids: Sequence[int], *, max_new_tokens: int,
                 reserve_steps: int = 16) -> None:
        if max_new_tokens < 0:
            raise ValueError("max_new_tokens must be >= 0")
        if reserve_steps <= 0:
            raise ValueError("reserve_steps must be positive")
        self.allocator = allocator
        self.request_ids = [int(r) for r in request_ids]
        if not self.request_ids:
            raise ValueError("DecodeBatch needs at least one request")
        if len(set(self.request_ids)) != len(self.request_ids):
            raise ValueError("request_ids must be distinct")
        self._requests = [allocator._get_request(r) for r in self.request_ids]
        self.device = allocator.device
        self.page = allocator.block_size
        self.max_new_tokens = int(max_new_tokens)
        self.reserve_steps = int(reserve_steps)
        self.steps_done = 0
        self._reserved_steps = 0
        self._taken: list[int] = []  # pages reserved by this batch, in the order taken
        self.host_lengths = [r.length for r in self._requests]
        cols = max(1, max((L + self.max_new_tokens + self.page - 1) // self.page for L in self.host_lengths))
        self._table_host = np.full((len(self._requests), cols), -1, dtype=np.int32)
        for i, r in enumerate(self._requests):
            self._table_host[i, : len(r.logical_blocks)] = r.logical_blocks
        try:
            self._reserve(min(self.max_new_tokens, self.reserve_steps))
        except BaseException:
            self._unreserve_all()
            raise
        self.block_table = torch.empty((len(self._requests), cols), dtype=torch.int32, device=self.device)
        self._upload_table()
        lengths = torch.tensor(self.host_lengths, dtype=torch.int64)
        self._lengths = [lengths.to(self.device), lengths.to(self.device).clone()]
        self._cur = 0
        self._caches: dict = {}  # lengths buffer -> ((buffer, max_seq_len), PagedKVCache)
        # Longest requests first: the decode's workgroups start with the longest rows, so its last
        # round holds short ones (every request grows by one token per step, so the order holds
        # for the batch's life).  Measured on MI355X, 64 ragged requests: 600 instead of 611 us.
        order = sorted(range(len(self._requests)), key=lambda i: -self.host_lengths[i])
        self._order = torch.tensor(order, dtype=torch.int32).to(self.device)
        # appended tokens that found no page (a -1 table entry): counted on the device by the append
        # kernels, checked at close() (the reference allocator raises instead, paged.py:89-90, 222-224)
        self._dropped = torch.zeros(1, dtype=torch.int32, device=self.device)
        self._open = True

    # -- bookkeeping ----------------------------------------------------------------------
    @property
    def lengths(self) -> torch.Tensor:
        return self._lengths[self._cur]

    def _reserve(self, upto_step: int) -> None:
        for s in range(self._reserved_steps, upto_step):
            for i, r in enumerate(self._requests):
                pos = self.host_lengths[i] + (s - self.steps_done)
                lp = pos // self.page
                if lp == len(r.logical_blocks):
                    pg = self.allocator._allocate_block()
                    r.logical_blocks.append(pg)
                    self._taken.append(pg)
                    self._table_host[i, lp] = pg
        self._reserved_steps = max(self._reserved_steps, upto_step)

    def _unreserve_all(self) -> None:
        """Undo every reservation of this batch (a failed first reservation): the pages leave their
        requests and go back to the front of the free list in the order they were taken."""

        taken = set(self._taken)
        for r in self._requests:
            r.logical_blocks[:] = [pg for pg in r.logical_blocks if pg not in taken]
        self.allocator._free_blocks[:0] = self._taken
        self._taken = []
        self._reserved_steps = 0

    def _upload_table(self) -> None:
        src = torch.from_numpy(self._table_host)
        if self.device.type == "cuda":
            self.block_table.copy_(src.pin_memory(), non_blocking=True)
        else:
            self.block_table.copy_(src)

    def cache(self) -> PagedKVCache:
        """The batch as a PagedKVCache over the current lengths buffer.

        ``max_seq_len`` is the longest request rounded up to a whole page (the kernels mask by the
        device lengths, and the table covers every page the batch reserved), so the same two
        objects -- one per lengths buffer -- serve up to ``page`` steps in a row and the launch
        path's layout validation memo holds across those steps."""

        cap = -(-max(1, max(self.host_lengths)) // self.page) * self.page
        key = (self._cur, cap)
        cached = self._caches.get(self._cur)
        if cached is None or cached[0] != key:
            cached = (key, PagedKVCache(k_quant=self.allocator.k_quant, v_quant=self.allocator.v_quant,
                                        block_table=self.block_table, lengths=self.lengths, block_size=self.page,
                                        max_seq_len=cap))
            self._caches[self._cur] = cached
        return cached[1]

    # -- decode ---------------------------------------------------------------------------
    def append(self, k_new: torch.Tensor, v_new: torch.Tensor) -> None:
        """Append ``k_new``/``v_new`` ``[n, heads, 1, head_dim]`` (one token per request)."""

        if not self._open:
            raise RuntimeError("DecodeBatch is closed")
        if self.steps_done >= self.max_new_tokens:
            raise RuntimeError(f"DecodeBatch was opened for {self.max_new_tokens} new tokens")
        n, a = len(self._requests), self.allocator
        for t in (k_new, v_new):
            if t.shape != (n, a.heads, 1, a.head_dim):
                raise ValueError(f"expected new K/V of shape {(n, a.heads, 1, a.head_dim)}, got {tuple(t.shape)}")
            if t.device != self.device:
                raise ValueError("new K/V must be on the allocator's device")
        if self.steps_done >= self._reserved_steps:
            self._reserve(min(self.max_new_tokens, self.steps_done + self.reserve_steps))
            self._upload_table()
        nxt = 1 - self._cur
        if self.device.type == "cuda":
            self._append_hip(k_new, v_new, self._lengths[self._cur], self._lengths[nxt])
        else:
            self._append_portable(k_new, v_new)
            self._lengths[nxt].copy_(self._lengths[self._cur] + 1)
        self._cur = nxt
        self.steps_done += 1
        for i, r in enumerate(self._requests):
            self.host_lengths[i] += 1
            r.length += 1

    def _append_hip(self, k_new, v_new, len_in, len_out) -> None:
        lib = _lib.require()
        if k_new.dtype != v_new.dtype:
            raise ValueError("k_new and v_new must share a dtype")
        k_c, v_c = k_new.contiguous(), v_new.contiguous()
        ks, vs = self.allocator.k_quant, self.allocator.v_quant
        _lib.check(lib.fs_append_tokens_i8(
            k_c.data_ptr(), v_c.data_ptr(), _lib.dtype_code(k_c.dtype), ks.values.data_ptr(), ks.scale.data_ptr(),
            ks.zero_point.data_ptr(), vs.values.data_ptr(), vs.scale.data_ptr(), vs.zero_point.data_ptr(),
            int(ks.values.shape[0]), self.block_table.data_ptr(), 4, int(self.block_table.shape[1]),
            len_in.data_ptr(), len_out.data_ptr(), len(self._requests), self.allocator.heads,
            self.allocator.head_dim, self.page, self._dropped.data_ptr(), _lib.stream_ptr(k_c.device)))

    def _append_portable(self, k_new, v_new) -> None:
        pos = torch.tensor(self.host_lengths, dtype=torch.int64)
        pages = torch.from_numpy(self._table_host[np.arange(len(self._requests)), (pos // self.page).numpy()])
        pages = pages.to(torch.int64)
        rows = torch.arange(len(self._requests))
        for store, src in ((self.allocator.k_quant, k_new), (self.allocator.v_quant, v_new)):
            sub = QuantizedTensor(store.values[pages], store.scale[pages], store.zero_point[pages], self.page,
                                  (len(pages), self.allocator.heads, self.page, self.allocator.head_dim))
            block = dequantize_int8_per_block(sub, dtype=torch.float32)
            block[rows, :, pos % self.page, :] = src[:, :, 0, :].to(torch.float32)
            q = quantize_int8_per_block(block, block_size=self.page)
            store.values[pages] = q.values
            store.scale[pages] = q.scale
            store.zero_point[pages] = q.zero_point

    def attend(self, q: torch.Tensor, *, return_stats: bool = False):
        """Paged INT8 decode attention of ``q [n, heads, head_dim]`` over the current cache (on GPU
        with the requests dispatched longest first; the output does not depend on the order)."""

        if q.device.type == "cuda" and q.device == self.device:
            from .triton_paged import _run_paged_quant_attention_triton

            return _run_paged_quant_attention_triton(q, self.cache(), return_stats=return_stats,
                                                     request_order=self._order)
        return paged_quant_attention_triton(q, self.cache(), return_stats=return_stats)

    def step(self, q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor) -> torch.Tensor:
        """One serving decode step: append one token per request, then attend over the updated cache.

        On GPU, with 16-token pages, head_dim 64 / 128 / 256, q, k_new, v_new of one dtype, and a
        decode grid of at most one workgroup per CU, both happen in one launch
        (``fs_paged_decode_append_i8``: the append runs inside the decode kernel and gives the same
        pages, lengths and output, bit for bit, as ``append`` followed by ``attend``).  Otherwise
        the two run one after the other: there the wave that requantizes a request's page holds up
        its workgroup's closing barrier, once per round of workgroups on a CU, which costs more
        than the separate append launch.  Measured on MI355X (H32 D128, ragged lengths, shuffled
        pool), one launch / two launches: B4 29.1 / 32.6 us, B16 69.3 / 68.8 us, B64 639 / 635 us."""

        if self._fusable(q, k_new, v_new):
            plan = self._fused_plan(q)
            if plan is not None:
                return self._step_fused(q, k_new, v_new, plan)
        self.append(k_new, v_new)
        return self.attend(q)

    def _fusable(self, q, k_new, v_new) -> bool:
        a = self.allocator
        return (self._open and self.device.type == "cuda" and self.page == 16 and a.k_quant.block_size == 16
                and a.head_dim in (64, 128, 256) and q.dtype == k_new.dtype == v_new.dtype
                and tuple(q.shape) == (len(self._requests), a.heads, a.head_dim) and q.device == self.device
                and self.steps_done < self.max_new_tokens)

    def _fused_plan(self, q):
        """(max_seq_len, launch plan) of a one-launch step whose grid fits one workgroup per CU, else None."""

        from .triton_utils import device_cu_count, launch_plan

        a = self.allocator
        # every row covers its appended token: the longest request after the step, in whole pages
        max_seq_len = -(-(max(self.host_lengths) + 1) // self.page) * self.page
        rows = len(self._requests) * a.heads
        plan = launch_plan(max_seq_len, rows, a.head_dim, self.page, self.page, self.device,
                           light=q.dtype in (torch.float16, torch.bfloat16))
        if rows * plan[3] > device_cu_count(self.device):
            return None
        return max_seq_len, plan

    def _step_fused(self, q, k_new, v_new, fused_plan) -> torch.Tensor:
        from .triton_utils import MERGE_MAX_WAVES, merge_area

        n, a = len(self._requests), self.allocator
        for t in (k_new, v_new):
            if t.shape != (n, a.heads, 1, a.head_dim):
                raise ValueError(f"expected new K/V of shape {(n, a.heads, 1, a.head_dim)}, got {tuple(t.shape)}")
            if t.device != self.device:
                raise ValueError("new K/V must be on the allocator's device")
        if self.steps_done >= self._reserved_steps:
            self._reserve(min(self.max_new_tokens, self.steps_done + self.reserve_steps))
            self._upload_table()
        lib = _lib.require()
        q_c, k_c, v_c = q.contiguous(), k_new.contiguous(), v_new.contiguous()
        ks, vs = a.k_quant, a.v_quant
        max_seq_len, (tiled, waves, split_tiles, max_splits, _) = fused_plan
        rows = n * a.heads
        out = torch.empty_like(q_c)
        area, area_bytes, workspace, ws_bytes = None, 0, None, 0
        if max_splits > 1 and waves <= MERGE_MAX_WAVES:
            area, area_bytes = merge_area(self.device, rows, max_splits, a.head_dim)
        elif max_splits > 1:
            ws_bytes = int(lib.fs_decode_workspace_bytes(rows, max_splits, a.head_dim))
            workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=self.device)
        nxt = 1 - self._cur
        _lib.check(lib.fs_paged_decode_append_i8(
            q_c.data_ptr(), _lib.dtype_code(q_c.dtype), k_c.data_ptr(), v_c.data_ptr(), ks.values.data_ptr(),
            ks.scale.data_ptr(), ks.zero_point.data_ptr(), vs.values.data_ptr(), vs.scale.data_ptr(),
            vs.zero_point.data_ptr(), self.block_table.data_ptr(), 4, int(self.block_table.shape[1]),
            self._lengths[self._cur].data_ptr(), self._lengths[nxt].data_ptr(), out.data_ptr(), _lib.ptr(workspace),
            ws_bytes, _lib.ptr(area), area_bytes, n, a.heads, a.head_dim, int(ks.values.shape[0]), self.page,
            max_seq_len, 1.0 / math.sqrt(a.head_dim), split_tiles, max_splits, waves, self._dropped.data_ptr(),
            _lib.stream_ptr(self.device)))
        self._cur = nxt
        self.steps_done += 1
        for i, r in enumerate(self._requests):
            self.host_lengths[i] += 1
            r.length += 1
        return out

    def dropped_tokens(self) -> int:
        """Appended tokens that found no page (block table entry -1 or past the table) and were
        dropped by the device append, since the batch opened (reads the device counter: a sync)."""

        return int(self._dropped.item())

    def close(self) -> None:
        """Return reserved pages that hold no token to the front of the free list, in taken order.

        Raises RuntimeError afterwards if any appended token was dropped for want of a page (the
        reference allocator raises when it has no page for a token, paged.py:89-90, 222-224)."""

        if not self._open:
            return
        unused = []
        for r in self._requests:
            need = (r.length + self.page - 1) // self.page
            unused.extend(r.logical_blocks[need:])
            del r.logical_blocks[need:]
        unused_set = set(unused)
        self.allocator._free_blocks[:0] = [p for p in self._taken if p in unused_set]
        self._open = False
        dropped = self.dropped_tokens()
        if dropped:
            raise RuntimeError(f"DecodeBatch: {dropped} appended token(s) found no page and were dropped")


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
