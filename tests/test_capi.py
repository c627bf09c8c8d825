"""The C-ABI library loads and exports every entry point include/flashspec_hip.h declares.

CPU only: nothing here launches a kernel.  Argument validation happens before
any HIP call, so rejected calls are safe without a GPU.
"""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from flashspec_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "flashspec_hip.h"


def declared_symbols() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fs_[a-z0-9_]+)\s*\(", text)))


def test_library_loads():
    assert _lib.available(), _lib.LOAD_ERROR


def test_every_declared_symbol_is_exported_and_bound():
    lib = ctypes.CDLL(str(_lib.LIB_PATH))
    names = declared_symbols()
    assert "fs_paged_decode_i8" in names and "fs_fused_decode_i8" in names
    for name in names:
        assert hasattr(lib, name), f"{name} not exported"
        assert name in _lib._SIGNATURES, f"{name} has no ctypes signature"


def test_abi_version_and_workspace_size():
    lib = _lib.require()
    assert lib.fs_abi_version() == 2
    assert lib.fs_decode_workspace_bytes(256, 16, 128) == 256 * 16 * 130 * 4


def test_invalid_arguments_are_rejected_before_launch():
    lib = _lib.require()
    # head_dim 0 -> FS_ERR_INVALID, message names the problem
    rc = lib.fs_paged_decode_i8(1, 1, 1, 1, 1, 1, 1, 1, 1, 8, 4, 1, 1, None, 0, 1, 1, 0, 4, 16, 16, 64,
                                0.1, 4, 1, 4, None)
    assert rc == _lib.FS_ERR_INVALID
    assert "head_dim" in lib.fs_last_error().decode()
    with pytest.raises(ValueError):
        _lib.check(rc)
    # splits that do not cover the sequence
    rc = lib.fs_fused_decode_i8(1, 1, 1, 1, 1, 1, 1, 1, None, 1, None, 0, 1, 1, 128, 4096, 256, 16, 0.1,
                                4, 4, 4, None)
    assert rc == _lib.FS_ERR_INVALID and "cover" in lib.fs_last_error().decode()
    # tiled path: more than 64 tiles per wave in one split
    rc = lib.fs_fused_decode_i8(1, 1, 1, 1, 1, 1, 1, 1, None, 1, None, 0, 1, 1, 128, 4096, 256, 16, 0.1,
                                256, 1, 2, None)
    assert rc == _lib.FS_ERR_INVALID and "64" in lib.fs_last_error().decode()
    assert lib.fs_decode_tiled_path(128, 16, 16) == 1 and lib.fs_decode_tiled_path(128, 32, 16) == 1
    assert lib.fs_decode_tiled_path(48, 16, 16) == 1 and lib.fs_decode_tiled_path(96, 32, 32) == 1
    assert lib.fs_decode_tiled_path(128, 16, 8) == 1 and lib.fs_decode_tiled_path(128, 24, 24) == 1
    assert lib.fs_decode_tiled_path(128, 4, 4) == 0 and lib.fs_decode_tiled_path(66, 16, 16) == 0
    # head_dim a multiple of 4 but not of 16 (>= 20): block and per-token parameters on the tiled path
    assert lib.fs_decode_tiled_path(72, 16, 16) == 1 and lib.fs_decode_tiled_path(24, 16, 1) == 1
    assert lib.fs_decode_tiled_path(68, 16, 16) == 1 and lib.fs_decode_tiled_path(36, 32, 1) == 1
    assert lib.fs_decode_tiled_path(20, 16, 16) == 1 and lib.fs_decode_tiled_path(252, 16, 16) == 1
    assert lib.fs_decode_tiled_path(8, 16, 16) == 0 and lib.fs_decode_tiled_path(12, 16, 16) == 0
    assert lib.fs_decode_tiled_path(72, 8, 8) == 0 and lib.fs_decode_tiled_path(36, 8, 8) == 0
    assert lib.fs_decode_tiled_path(34, 16, 16) == 0 and lib.fs_decode_tiled_path(260, 16, 16) == 0
    assert lib.fs_decode_tiled_path_channel(72, 16, 16) == 0 and lib.fs_decode_tiled_path_channel(36, 16, 16) == 0
    assert lib.fs_decode_tiled_path(128, 48, 32) == 0 and lib.fs_decode_tiled_path(512, 16, 16) == 0
    # per-channel stores with 64-token blocks: waves take whole blocks, so a split holds whole
    # blocks of 4 tiles and a wave at most 64 tiles
    rc = lib.fs_fused_decode_i8_channel(1, 1, 1, 1, 1, 1, 1, 1, None, 1, 1, 1 << 20, 1, 1, 128, 4096, 64, 64,
                                        0.1, 30, 9, 8, None)
    assert rc == _lib.FS_ERR_INVALID and "multiple of quant_block / 16" in lib.fs_last_error().decode()
    # 48-token blocks: 85 blocks over 4 waves is 22 blocks = 66 tiles for the first wave
    rc = lib.fs_fused_decode_i8_channel(1, 1, 1, 1, 1, 1, 1, 1, None, 1, None, 0, 1, 1, 128, 4080, 85, 48,
                                        0.1, 255, 1, 4, None)
    assert rc == _lib.FS_ERR_INVALID and "<= 64" in lib.fs_last_error().decode()
    assert lib.fs_decode_tiled_path_channel(128, 64, 64) == 1 and lib.fs_decode_tiled_path_channel(128, 8, 8) == 0
    assert lib.fs_decode_tiled_path_channel(128, 2048, 2048) == 0  # a block of more than 64 tiles
    # nodes per workgroup of the multi-query tree kernel: 32 where a wave has registers for two
    # 16-node groups and 16-node workgroups would not fit the CUs in one round
    npw = lib.fs_tree_nodes_per_workgroup
    f32, f16, bf16 = 0, 1, 2  # FS_F32, FS_F16, FS_BF16
    assert npw(128, 16, f16, 16, 128, 256) == 16 and npw(128, 17, f16, 16, 128, 256) == 16
    assert npw(128, 17, f16, 16, 129, 256) == 32 and npw(128, 64, bf16, 16, 128, 256) == 32
    assert npw(64, 64, f32, 1, 128, 256) == 32 and npw(128, 32, f16, 16, 128, 256) == 16
    assert npw(128, 64, f32, 16, 128, 256) == 16 and npw(128, 64, f16, 1, 128, 256) == 16
    assert npw(256, 64, f16, 16, 128, 256) == 16
    # unsupported dtype code in quantize
    rc = lib.fs_quantize_i8(1, 9, 1, 16, 128, 16, 1, 1, 1, None)
    assert rc == _lib.FS_ERR_INVALID
    # in-place page update with a different quant block
    rc = lib.fs_update_pages_i8(1, 1, 1, 4, 8, 1, 1, 1, None, None, 4, 1, 1, 0, 1, 2, 16, 64, None)
    assert rc == _lib.FS_ERR_INVALID and "in-place" in lib.fs_last_error().decode()
    # append: the two lengths buffers must differ, and the table index width is 4 or 8 bytes
    rc = lib.fs_append_tokens_i8(1, 1, 1, 1, 1, 1, 1, 1, 1, 8, 1, 8, 4, 7, 7, 2, 2, 64, 16, None, None)
    assert rc == _lib.FS_ERR_INVALID and "differ" in lib.fs_last_error().decode()
    rc = lib.fs_append_tokens_i8(1, 1, 1, 1, 1, 1, 1, 1, 1, 8, 1, 2, 4, 7, 9, 2, 2, 64, 16, None, None)
    assert rc == _lib.FS_ERR_INVALID and "int32 or int64" in lib.fs_last_error().decode()
    # fused append + decode: 16-token pages, head_dim 64 / 128 / 256, two lengths buffers

    def fused(page, D, lens_in, lens_out):
        return lib.fs_paged_decode_append_i8(1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 1, 8, 4, lens_in, lens_out, 1, None, 0,
                                             None, 0, 2, 2, D, 8, page, 64, 0.1, 4, 1, 1, None, None)

    assert fused(32, 128, 7, 9) == _lib.FS_ERR_INVALID and "16-token pages" in lib.fs_last_error().decode()
    assert fused(16, 96, 7, 9) == _lib.FS_ERR_INVALID and "64, 128 or 256" in lib.fs_last_error().decode()
    assert fused(16, 128, 7, 7) == _lib.FS_ERR_INVALID and "lengths_out" in lib.fs_last_error().decode()
    assert fused(16, 128, 7, None) == _lib.FS_ERR_INVALID
    # a request order needs the tiled path (head_dim 34 takes the generic kernel)
    rc = lib.fs_paged_decode_ordered(1, 1, 1, 1, 1, 1, 1, 1, 1, 8, 4, 1, 1, 1, None, 0, None, 0, 2, 2, 34, 8, 16, 16,
                                     64, 0.1, 4, 1, 1, None)
    assert rc == _lib.FS_ERR_INVALID and "tiled" in lib.fs_last_error().decode()
    # tree verification with the in-launch merge: INT8 or FP8 only, 16 / 32 / library-chosen node groups,
    # the multi-query kernel's shapes
    tree = lib.fs_tree_verify_merged

    def merged(kv_format=0, npw=0, head_dim=128, max_splits=1, area=None, area_bytes=0):
        return tree(1, 1, kv_format, 1, 1, 1, 1, 1, 1, 1, 8, 4, 1, 1, 1, 1, 1, area, area_bytes, 2, 4, 2, head_dim, 8,
                    16, 16, 64, 0.1, 4, max_splits, 8, npw, None)

    assert merged(kv_format=2) == _lib.FS_ERR_INVALID and "kv_format" in lib.fs_last_error().decode()
    assert merged(npw=8) == _lib.FS_ERR_INVALID and "nodes_per_workgroup" in lib.fs_last_error().decode()
    assert merged(head_dim=96) == _lib.FS_ERR_INVALID and "multi-query" in lib.fs_last_error().decode()
    # the in-launch merge keeps 2 floats per node and split in its LDS accumulator buffer: at most
    # 272 splits at head_dim 64 (a 256-aligned stand-in address; rejected before any HIP call)
    assert merged(npw=16, head_dim=64, max_splits=273, area=256, area_bytes=1 << 40) == _lib.FS_ERR_INVALID
    assert "at most 272 splits" in lib.fs_last_error().decode()
    from flashspec_amd.triton_utils import plan_tree_splits, tree_merge_max_splits

    assert [tree_merge_max_splits(d) for d in (64, 128, 256)] == [272, 528, 520]
    assert plan_tree_splits(1 << 20, 1, 64, 1 << 12)[1] <= 272


def test_no_alloc_entry_point_rejects_plans_beyond_its_array():
    """fs_paged_decode_i8_noalloc checks the partials' size against its per-GPU array before any
    HIP call (no GPU needed)."""

    lib = _lib.require()
    assert lib.fs_noalloc_scratch_bytes() == 16 << 20
    # 256 rows x 1024 splits x (128 + 2) floats = 136 MB of partials
    rc = lib.fs_paged_decode_i8_noalloc(1, 1, 1, 1, 1, 1, 1, 1, 1, 8, 4, 1, 1, 8, 32, 128, 64, 16, 16, 16384,
                                        0.1, 1, 1024, 1, None)
    assert rc == _lib.FS_ERR_INVALID and "at most" in lib.fs_last_error().decode()
    rc = lib.fs_paged_decode_i8_noalloc(1, 1, 1, 1, 1, 1, 1, 1, 1, 8, 4, 1, 1, 0, 32, 128, 64, 16, 16, 16384,
                                        0.1, 1, 2, 1, None)
    assert rc == _lib.FS_ERR_INVALID
