"""Backend gate, dispatch and launch knobs (reference src/flashspec/triton_utils.py).

The reference gates its GPU path on ``HAS_TRITON``.  Here the accelerated
backend is the HIP library, so ``HAS_TRITON`` (alias ``HAS_HIP``) means
"libflashspec_hip.so is loaded".  Dispatch keeps the reference's contract —
GPU path when the first positional argument is a GPU tensor, portable torch
path otherwise — except that a GPU tensor with the library missing raises
instead of silently running the portable path.
"""

from __future__ import annotations

import functools
import math
import os

from . import _lib

HAS_HIP = _lib.available()
HAS_TRITON = HAS_HIP  # name kept for callers of the reference (tests, microbench)

TILE_TOKENS = 16  # tokens per decode tile / quant block on the fast path


def next_power_of_2(x: int) -> int:
    return 1 << (x - 1).bit_length()


def validate_decode_query(q, *, kernel_name: str) -> None:
    """Query checks shared by both kernels (triton_utils.py:33-45)."""

    if q.ndim != 3:
        raise ValueError("q must be [batch, heads, head_dim]")
    if q.device.type != "cuda":
        raise RuntimeError(f"HIP {kernel_name} attention needs a GPU q tensor")
    if q.shape[-1] > 256:
        raise ValueError(f"HIP {kernel_name} attention supports head_dim <= 256")


def dispatch_triton_or_fallback(args, kwargs, *, run_triton, load_fallback, extra_guard=None):
    """GPU path iff ``args[0]`` is a GPU tensor and ``extra_guard(args)`` holds (triton_utils.py:48-73).

    A GPU call without the HIP library raises RuntimeError rather than falling back.
    """

    import torch

    if args and isinstance(args[0], torch.Tensor) and args[0].device.type == "cuda" and (
        extra_guard is None or extra_guard(args)
    ):
        _lib.require()
        return run_triton(*args, **kwargs)
    return load_fallback()(*args, **kwargs)


# ---- layout memo ----------------------------------------------------------------------------
# The K/V containers (QuantizedTensor, PagedKVCache) are frozen dataclasses: their tensors
# never change identity.  After a full validation, the container remembers the query
# signature (shape, dtype, device) and companions it was checked with, plus the data
# pointers and element counts of its tensors, so repeated launches over the same cache skip
# the checks (about 10 us of host time per call).  Any difference, including a tensor resized
# in place, re-runs the full validation.
_MEMO_ATTR = "_fs_layout_checked"


def layout_checked(owner, key) -> bool:
    """True when ``owner`` passed validation before with this exact ``key``."""

    return owner.__dict__.get(_MEMO_ATTR) == key


def remember_layout(owner, key) -> None:
    object.__setattr__(owner, _MEMO_ATTR, key)


# ---- merge areas of the in-kernel split merge -----------------------------------------------
# Rows that split merge inside the decode launch: the last split of a row to finish merges it,
# through a merge area that must be all zero before a launch and that every launch leaves all zero
# again.  One zero-filled area per (device, stream) serves every eager call on that stream, grown
# when a launch needs more.  Under stream capture each call zero-fills an area of its own inside
# the capture (a fill kernel, recorded with the decode), so every replay starts from zero without
# sharing memory with eager calls.
_MERGE_AREAS: dict = {}
_MERGE_AREA_MIN_BYTES = 1 << 16
# Split launches of up to this many waves per workgroup merge in-kernel; 16-wave workgroups keep
# the workspace + merge-launch path.  Measured on MI355X (paged, H32 D128, same box), in-kernel /
# two launches / decode alone, us: B4 S2048 2 splits x 4 waves 16.46 / 18.15 / 14.55, B4 S4096
# 2 x 4 26.13 / 27.86 / 24.56, B2 S8192 4 x 4 26.44 / 27.70 / 24.24, B1 S16384 8 x 4 28.08 / 28.81 /
# 24.36; B2 S8192 8 x 16 35.32 / 33.71 / 29.23.
MERGE_MAX_WAVES = 8


@functools.lru_cache(maxsize=256)
def _merge_area_bytes(rows: int, max_splits: int, head_dim: int) -> int:
    return int(_lib.require().fs_decode_merge_area_bytes(rows, max_splits, head_dim))


def merge_area(device, rows: int, max_splits: int, head_dim: int, stream: int | None = None):
    """(tensor, bytes) of a zero-filled merge area for one decode launch on the current stream
    (``stream``: its handle, when the caller has it already)."""

    import torch

    need = _merge_area_bytes(rows, max_splits, head_dim)
    if torch.cuda.is_current_stream_capturing():
        area = torch.zeros(need, dtype=torch.uint8, device=device)
        return area, need
    dev = torch_device(device)
    index = dev.index if dev.index is not None else torch.cuda.current_device()
    key = (index, stream if stream is not None else _lib.stream_ptr(dev))
    area = _MERGE_AREAS.get(key)
    if area is None or area.numel() < need:
        area = torch.zeros(max(need, _MERGE_AREA_MIN_BYTES), dtype=torch.uint8, device=device)
        _MERGE_AREAS[key] = area
    return area, int(area.numel())


def kv_format_code(per_channel: bool, fp8: bool) -> int:
    """kv_format of the merged decode entry points: 0 affine INT8, 1 FP8 E4M3, 2 per-channel INT8."""

    return 2 if per_channel else (1 if fp8 else 0)


_DEFAULT_BLOCK_N = 128


def resolve_block_n() -> int:
    """Tokens per tile knob, default 128, ``FLASHSPEC_BLOCK_N`` in {16,32,64,128} (triton_utils.py:81-98).

    The HIP kernels always stream 16-token tiles; block_n is the granularity the
    ``FLASHSPEC_NUM_SPLITS`` override is clamped with, as in the reference.
    """

    override = os.environ.get("FLASHSPEC_BLOCK_N")
    if override is not None:
        try:
            v = int(override)
        except ValueError:
            v = 0
        if v in (16, 32, 64, 128):
            return v
    return _DEFAULT_BLOCK_N


def resolve_num_warps() -> int:
    """Waves per workgroup, default 4, ``FLASHSPEC_NUM_WARPS`` in {1,2,4,8} (triton_utils.py:101-116)."""

    override = os.environ.get("FLASHSPEC_NUM_WARPS")
    if override is not None:
        try:
            v = int(override)
        except ValueError:
            v = 0
        if v in (1, 2, 4, 8):
            return v
    return 4


# ---- split-K planning for the HIP kernels ---------------------------------------------------
# Tiled path: one split = one workgroup of W cooperating waves.  Rows split only when
# there are fewer rows than CUs (the split count fills the GPU, each split keeping at
# least MIN_SPLIT_TILES tiles); W is then the largest power of two up to 16 that leaves
# every wave MIN_TILES_PER_WAVE tiles, unless FLASHSPEC_NUM_WARPS fixes it.  A split
# holds at most 64 tiles per wave.  Generic path: one split = one wave of 8..64 tiles.
MAX_TILED_WAVES = 16
MIN_SPLIT_TILES = 8
MIN_TILES_PER_WAVE = 4
MAX_TILES_PER_WAVE = 64
# Light tiles (fp16 or bf16 query, INT8 or FP8 E4M3 values with one scale (and zero point) per
# 16-token page, head_dim 128: the fp16 dot2 score path with every lane busy; bf16 rows enter it
# scaled by a power of two) run 4-wave workgroups when the grid puts one workgroup on 3/4 to all of
# the CUs and a split holds 128..256 tiles (32..64 per wave, so no extra split).  Measured on MI355X
# (one box each, settled clocks, 3 rotated input sets), paged / fused us with 4 against 16 waves:
# B8 H32 S4096 D128 43.4 / 42.1 vs 45.5 / 43.1 (bf16 query: 41.6-41.7 / 41.0-41.1 vs 44.2 /
# 42.9-43.8; FP8 values: 43.5-44.2 / 40.9-41.1 vs 44.1-44.3 / 44.2-44.4), S2048 25.1 / 24.3 vs
# 26.4 / 24.8, B4 S8192 46.4 / 45.0 vs 49.0 / 46.3, B2 S8192 29.3 / 27.3 vs 30.1 / 27.8, B1 S16384
# 29.7 / 29.2 vs 30.4 / 29.3.  Heavier tiles (fp32 query,
# per-token or per-channel parameters, 64- or 256-dim layouts, head_dim 96 in the 128-dim layout:
# 41.0 vs 37.5 us, pages of two quant blocks: 45.2 vs 44.5 us) and grids of more than one
# workgroup per CU (ragged B16: 56.5 vs 49.7 us) keep more waves, and so do half-empty grids
# (B4 S2048 in one split: 21.8 us with 4 waves, 18.2 with 8, 19.3 with 16).
# Splits of 64..127 light tiles take 4 waves as well, with the in-kernel split merge: measured on
# MI355X (paged H32 D128, one box, direct C-ABI loop), B4 S2048 (C1, 128 rows of 128 tiles) 2 splits
# x 4 waves merged 16.48 us against 17.67 unsplit x 8 (the plan before) and 18.33 for 2 x 4 with the
# merge launch; B2 S4096 4 x 4 merged 17.52 against 20.62 for 4 x 16 with the merge launch.
LIGHT_WAVES = 4
LIGHT_MIN_SPLIT_TILES = 64
# Rows that fill at least half of the CUs split in two only when each half keeps 128 tiles (light
# tiles: LIGHT_MIN_SPLIT_TILES); otherwise they run unsplit with at most 8 waves per workgroup.
# Measured on MI355X before the in-kernel merge, B4 H32 S2048 D128 (fp16 query), paged / fused us:
# unsplit x 8 waves 18.2 / 17.6, unsplit x 16 19.3 / 18.0, 2 splits x 16 19.1 / 18.4;
# B4 S4096 (256 tiles) keeps its split: 2 x 4 waves 29.1 / 27.9 against unsplit x 8 29.9 / 29.3.
HALVE_MIN_SPLIT_TILES = 128
HALF_EMPTY_WAVES = 8
# A forced split count (FLASHSPEC_NUM_SPLITS) of two or more can put several workgroups on each CU:
# the plan then halves its waves while a workgroup holds more than 8 (what the in-kernel merge
# serves) or, with more workgroups than CUs, the grid more than FORCED_WAVES_PER_CU waves per CU, as
# long as a split's tiles still fit its waves.
# Measured on MI355X (one box, fused / paged us, 3+ rotated input sets), with the waves the plan
# took before: B8 H32 S4096 D128 4 splits (the reference's C2 setting) 2 waves 46.1 / 47.9 against
# 16 waves 53.5 / 57.3, 2 splits 4 waves 44.0 / 46.0 against 16 waves 49.4 / 53.0, 8 splits 1 wave
# 52.5 / 51.1 against 8 waves 57.7 / 58.3; B8 S2048 4 splits 2 waves 27.1 / 26.8 against 8 waves
# 31.4 / 31.7; B4 S2048 4 splits 4 waves 16.2 / 16.0 against 8 waves 17.0 / 16.9; B1 S16384
# 4 splits 8 waves 29.4 / 30.4 against 16 waves 31.6 / 33.1, 16 splits 4 waves 29.5 / 31.4
# against 16 waves 32.8 / 36.4.
FORCED_WAVES_PER_CU = 8
FORCED_MAX_WAVES = 8

# Contiguous (fused) rows at head_dim 64 take at most 8 waves per workgroup in the default plan
# (the 64-dim register layout; paged rows and the head_dims below 64 that share the layout keep
# up to 16).  Measured on MI355X (H32, one box, fused us, default 16 waves -> 8): B8 S4096 INT8
# 25.02 -> 23.12, bf16 / fp32 queries 24.5 / 24.35 -> 23.2 / 22.95, FP8 24.14 -> 22.81, 32-token
# blocks 24.5 -> 23.0, per-token scales 26.5 -> 24.96, B2 S8192 (4 splits) 18.2 -> 15.58, B1 S16384
# (8 splits) 18.2 -> 17.15, B16 S4096 43.2 -> 43.2; paged B8 S4096 26.0 -> 26.4; fused head_dim 48
# 19.3 -> 20.7 and 40 19.03 -> 20.76.
CONTIGUOUS_D64_WAVES = 8
GENERIC_WAVES_PER_CU = 16
GENERIC_MIN_SPLIT_TILES = 8
GENERIC_MAX_SPLIT_TILES = 64

_CU_CACHE: dict = {}


def device_cu_count(device) -> int:
    import torch

    dev = torch.device(device)
    key = dev.index if dev.index is not None else torch.cuda.current_device()
    if key not in _CU_CACHE:
        _CU_CACHE[key] = int(torch.cuda.get_device_properties(key).multi_processor_count)
    return _CU_CACHE[key]


def forced_num_splits(seq_len: int, block_n: int) -> int | None:
    """``FLASHSPEC_NUM_SPLITS`` clamped to [1, ceil(seq_len/block_n)] (triton_fused.py:586-595)."""

    override = os.environ.get("FLASHSPEC_NUM_SPLITS")
    if override is None:
        return None
    try:
        forced = int(override)
    except ValueError:
        return None
    if forced < 1:
        return None
    max_splits = max(1, (seq_len + block_n - 1) // block_n)
    return max(1, min(forced, max_splits))


def forced_tiled_waves() -> int | None:
    """FLASHSPEC_NUM_WARPS as waves per workgroup on the tiled path (1/2/4/8/16), or None."""

    override = os.environ.get("FLASHSPEC_NUM_WARPS")
    if override is None:
        return None
    try:
        v = int(override)
    except ValueError:
        return None
    return v if v in (1, 2, 4, 8, 16) else None


def plan_splits(seq_len: int, rows: int, block_n: int, cu_count: int, *, tiled: bool = True,
                waves: int | None = None, max_waves: int = MAX_TILED_WAVES,
                tile_group: int = 1, light: bool = False) -> tuple[int, int, int]:
    """Return ``(split_tiles, max_splits, waves_per_block)`` for one decode launch.

    ``rows`` rows of up to ``seq_len`` tokens; ``waves`` fixes the workgroup size
    (tiled path) or the waves grouped per workgroup (generic path).  ``tile_group`` > 1
    (per-channel stores on the tiled path, quant_block / 16): waves take whole groups of that
    many tiles, so splits hold whole groups and a wave at most 64 tiles.  ``light``: the
    tiles take the fp16 dot2 score path (see LIGHT_WAVES).
    """

    tiles = max(1, math.ceil(seq_len / TILE_TOKENS))
    forced = forced_num_splits(seq_len, block_n)
    if tiled:
        grp = max(1, tile_group)
        groups = math.ceil(tiles / grp)
        half_empty = False
        if forced is not None:
            n = forced
        else:
            n = max(1, math.ceil(cu_count / max(1, rows)))
            n = min(n, max(1, math.ceil(tiles / MIN_SPLIT_TILES)))
            halve_min = LIGHT_MIN_SPLIT_TILES if light and grp == 1 else HALVE_MIN_SPLIT_TILES
            if n == 2 and tiles < 2 * halve_min:
                # half the CUs or more already hold a row: a two-way split saves less than its
                # merge costs unless each half keeps halve_min tiles
                n, half_empty = 1, True
        n = min(n, groups)
        split_groups = math.ceil(groups / n)
        if waves is None:
            per_wave = max(MIN_TILES_PER_WAVE, grp)
            waves = 1
            while waves < max_waves and 2 * waves * per_wave <= split_groups * grp:
                waves *= 2
            if half_empty and grp == 1:
                waves = min(waves, HALF_EMPTY_WAVES)
            if light and grp == 1 and cu_count * 3 // 4 <= rows * n <= cu_count and \
                    LIGHT_MIN_SPLIT_TILES <= split_groups <= LIGHT_WAVES * MAX_TILES_PER_WAVE:
                waves = LIGHT_WAVES
            if forced is not None and n > 1:
                need = math.ceil(split_groups / (MAX_TILES_PER_WAVE // grp))  # waves a split's tiles need
                several = rows * n > cu_count  # more than one workgroup per CU
                while waves // 2 >= need and (waves > FORCED_MAX_WAVES or
                                              several and rows * n * waves > cu_count * FORCED_WAVES_PER_CU):
                    waves //= 2
        cap = MAX_TILES_PER_WAVE // grp * waves
        if split_groups > cap:
            split_groups = math.ceil(groups / math.ceil(groups / cap))
        split_tiles = split_groups * grp
    else:
        if forced is not None:
            split_tiles = math.ceil(tiles / forced)
        else:
            want = math.ceil(rows * tiles / max(1, cu_count * GENERIC_WAVES_PER_CU))
            split_tiles = min(max(want, GENERIC_MIN_SPLIT_TILES), GENERIC_MAX_SPLIT_TILES, tiles)
        waves = waves or 4
    split_tiles = max(1, split_tiles)
    return split_tiles, math.ceil(tiles / split_tiles), waves


# One 8-wave workgroup of the multi-query kernel holds a CU (its ~140 registers per lane leave
# room for 3 waves per SIMD): the plan splits only while the grid fits one workgroup per CU.
# Measured on MI355X, B4 H32 S4096 D128, 16 nodes: 2 splits (256 workgroups) 33.5 us,
# 4 splits (two rounds) 45.6 us; 4 nodes: 27.6 vs 35.0 us.
TREE_WG_PER_CU = 1


def tree_max_waves(head_dim: int) -> int:
    """Waves per workgroup of the multi-query tree kernel: 8 (4 for head_dim 256)."""

    return 4 if head_dim > 128 else 8


def tree_merge_max_splits(head_dim: int) -> int:
    """Splits per row that the multi-query tree kernel's in-launch merge holds (its LDS accumulator
    buffer keeps two floats per node and split): 272 at head_dim 64, 528 at 128, 520 at 256."""

    dp = 64 if head_dim <= 64 else (128 if head_dim <= 128 else 256)
    return tree_max_waves(head_dim) * (dp + 4) // 2


def plan_tree_splits(seq_len: int, units: int, head_dim: int, cu_count: int) -> tuple[int, int, int]:
    """``(split_tiles, max_splits, waves_per_block)`` of the multi-query tree kernel.

    ``units`` = batch * heads * ceil(nodes / per_workgroup) workgroups per split, with
    ``per_workgroup`` from ``fs_tree_nodes_per_workgroup`` (16, or 32 for trees of more than 16
    nodes where registers allow).  Workgroups of 8 waves (4 for head_dim 256, whose register
    layout is twice as wide); as many splits as keep the grid within one workgroup per CU, at
    least two tiles per wave; ``FLASHSPEC_NUM_SPLITS`` / ``FLASHSPEC_NUM_WARPS`` override as for
    the decode plan.
    """

    tiles = max(1, math.ceil(seq_len / TILE_TOKENS))
    cap = tree_max_waves(head_dim)
    forced_waves = forced_tiled_waves()
    waves = min(forced_waves, cap) if forced_waves is not None else cap
    forced = forced_num_splits(seq_len, resolve_block_n())
    if forced is not None:
        n = forced
    else:
        n = max(1, (TREE_WG_PER_CU * cu_count) // max(1, units))
        n = min(n, max(1, tiles // (2 * waves)))
    n = min(n, tree_merge_max_splits(head_dim))
    split_tiles = math.ceil(tiles / n)
    limit = MAX_TILES_PER_WAVE * waves
    if split_tiles > limit:
        split_tiles = math.ceil(tiles / math.ceil(tiles / limit))
    return split_tiles, math.ceil(tiles / split_tiles), waves


_PLAN_KNOBS = ("FLASHSPEC_NUM_WARPS", "FLASHSPEC_BLOCK_N", "FLASHSPEC_NUM_SPLITS")


def launch_plan(seq_len: int, rows: int, head_dim: int, page_size: int, quant_block: int, device,
                per_channel: bool = False, light: bool = False, contiguous: bool = False):
    """(tiled, waves_per_block, split_tiles, max_splits, block_n) for one decode launch.

    ``light``: fp16 or bf16 query over INT8 or FP8 values (the caller's part of the LIGHT_WAVES condition;
    the store layout part is checked here).  ``contiguous``: rows of a contiguous store (the fused
    kernel), whose default plan at head_dim 64 takes at most CONTIGUOUS_D64_WAVES waves.

    The plan is a pure function of the shape, the device and the three env knobs, which are
    read on every call; it is computed once per distinct combination (a few microseconds of
    host time saved per launch)."""

    dev = torch_device(device)
    env = os.environ
    knobs = tuple(env.get(k) for k in _PLAN_KNOBS)
    return _launch_plan_cached(int(seq_len), int(rows), int(head_dim), int(page_size), int(quant_block),
                               dev.type, dev.index, bool(per_channel), bool(light), bool(contiguous), knobs)


def torch_device(device):
    import torch

    return device if isinstance(device, torch.device) else torch.device(device)


@functools.lru_cache(maxsize=512)
def _launch_plan_cached(seq_len: int, rows: int, head_dim: int, page_size: int, quant_block: int, dev_type: str,
                        dev_index, per_channel: bool, light: bool, contiguous: bool, knobs: tuple):
    """`knobs` only keys the cache: the helpers below read the same values from the environment."""

    import torch

    from . import _lib

    device = torch.device(dev_type, dev_index) if dev_index is not None else torch.device(dev_type)
    lib = _lib.require()
    if per_channel:
        tiled = bool(lib.fs_decode_tiled_path_channel(head_dim, page_size, quant_block))
    else:
        tiled = bool(lib.fs_decode_tiled_path(head_dim, page_size, quant_block))
    # register budget: the 256-dim register layout and per-channel parameters run 8 waves
    max_waves = 8 if head_dim > 128 or per_channel else MAX_TILED_WAVES
    waves = forced_tiled_waves() if tiled else resolve_num_warps()
    if tiled and waves is not None:
        waves = min(waves, max_waves)
    block_n = resolve_block_n()
    group = quant_block // TILE_TOKENS if tiled and per_channel else 1
    light = light and tiled and not per_channel and quant_block == TILE_TOKENS and page_size == TILE_TOKENS and \
        head_dim == 128
    # the default plan's ceiling (a forced wave count keeps only the register limit above)
    if contiguous and tiled and not per_channel and head_dim == 64:
        max_waves = min(max_waves, CONTIGUOUS_D64_WAVES)
    split_tiles, max_splits, waves = plan_splits(seq_len, rows, block_n, device_cu_count(device), tiled=tiled,
                                                 waves=waves, max_waves=max_waves, tile_group=group, light=light)
    return tiled, waves, split_tiles, max_splits, block_n
