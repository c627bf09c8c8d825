"""ctypes binding of libflashspec_hip.so (the C ABI declared in include/flashspec_hip.h).

The library is loaded once at import.  ``available()`` says whether it loaded;
``require()`` returns it or raises RuntimeError naming the load failure, so a
GPU call never silently falls back to another implementation.
"""

from __future__ import annotations

import ctypes
import os
from ctypes import c_float, c_int, c_int64, c_void_p
from pathlib import Path

import torch

# FLASHSPEC_HIP_LIB may name another build of the same library (e.g. a tuning variant).
LIB_PATH = Path(os.environ.get("FLASHSPEC_HIP_LIB") or Path(__file__).resolve().with_name("libflashspec_hip.so"))

FS_OK, FS_ERR_INVALID, FS_ERR_RUNTIME = 0, 1, 2
DTYPE_CODE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}

# (name, restype, argtypes) for every exported entry point.
_SIGNATURES = {
    "fs_last_error": (ctypes.c_char_p, []),
    "fs_abi_version": (c_int, []),
    "fs_decode_workspace_bytes": (c_int64, [c_int64, c_int64, c_int64]),
    "fs_decode_tiled_path": (c_int, [c_int, c_int, c_int]),
    "fs_fused_decode_i8": (
        c_int,
        [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
         c_void_p, c_int64, c_int, c_int, c_int, c_int, c_int, c_int, c_float, c_int, c_int, c_int, c_void_p],
    ),
    "fs_paged_decode_i8": (
        c_int,
        [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int64,
         c_void_p, c_void_p, c_void_p, c_int64, c_int, c_int, c_int, c_int64, c_int, c_int, c_int, c_float,
         c_int, c_int, c_int, c_void_p],
    ),
    "fs_decode_merge_area_bytes": (c_int64, [c_int64, c_int64, c_int64]),
    "fs_fused_decode_merged": (
        c_int,
        [c_void_p, c_int, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
         c_void_p, c_int64, c_int, c_int, c_int, c_int, c_int, c_int, c_float, c_int, c_int, c_int, c_void_p],
    ),
    "fs_paged_decode_merged": (
        c_int,
        [c_void_p, c_int, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int,
         c_int64, c_void_p, c_void_p, c_void_p, c_int64, c_int, c_int, c_int, c_int64, c_int, c_int, c_int, c_float,
         c_int, c_int, c_int, c_void_p],
    ),
    "fs_paged_decode_i8_noalloc": (
        c_int,
        [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int64,
         c_void_p, c_void_p, c_int, c_int, c_int, c_int64, c_int, c_int, c_int, c_float, c_int, c_int, c_int,
         c_void_p],
    ),
    "fs_noalloc_scratch_bytes": (c_int64, []),
    "fs_tree_verify_i8": (
        c_int,
        [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int64,
         c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_int64, c_int, c_int, c_int, c_int,
         c_int64, c_int, c_int, c_int, c_float, c_int, c_int, c_int, c_int, c_void_p],
    ),
    "fs_tree_verify_fp8": (
        c_int,
        [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int64, c_void_p, c_void_p,
         c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_int64, c_int, c_int, c_int, c_int, c_int64, c_int, c_int,
         c_int, c_float, c_int, c_int, c_int, c_int, c_void_p],
    ),
    "fs_tree_verify_i8_channel": (
        c_int,
        [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int64,
         c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_int64, c_int, c_int, c_int, c_int,
         c_int64, c_int, c_int, c_int, c_float, c_int, c_int, c_int, c_int, c_void_p],
    ),
    "fs_tree_verify_merged": (
        c_int,
        [c_void_p, c_int, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int,
         c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int, c_int, c_int, c_int,
         c_int64, c_int, c_int, c_int, c_float, c_int, c_int, c_int, c_int, c_void_p],
    ),
    "fs_tree_mfma_path": (c_int, [c_int, c_int, c_int]),
    "fs_tree_nodes_per_workgroup": (c_int, [c_int, c_int, c_int, c_int, c_int64, c_int]),
    "fs_quantize_i8_channel": (
        c_int, [c_void_p, c_int, c_int64, c_int, c_int, c_int, c_void_p, c_void_p, c_void_p, c_void_p]
    ),
    "fs_quantize_pages_i8_channel": (
        c_int,
        [c_void_p, c_int, c_int, c_int, c_int, c_int, c_int, c_void_p, c_int64, c_void_p, c_void_p, c_void_p,
         c_void_p],
    ),
    "fs_fused_decode_i8_channel": (
        c_int,
        [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
         c_void_p, c_int64, c_int, c_int, c_int, c_int, c_int, c_int, c_float, c_int, c_int, c_int, c_void_p],
    ),
    "fs_paged_decode_i8_channel": (
        c_int,
        [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int64,
         c_void_p, c_void_p, c_void_p, c_int64, c_int, c_int, c_int, c_int64, c_int, c_int, c_int, c_float,
         c_int, c_int, c_int, c_void_p],
    ),
    "fs_decode_tiled_path_channel": (c_int, [c_int, c_int, c_int]),
    "fs_stream_read": (c_int, [c_void_p, c_int64, c_void_p, c_int, c_void_p]),
    "fs_stream_copy_half": (c_int, [c_void_p, c_int64, c_void_p, c_int, c_void_p]),
    "fs_quantize_fp8": (c_int, [c_void_p, c_int, c_int64, c_int, c_int, c_int, c_void_p, c_void_p, c_void_p, c_void_p]),
    "fs_quantize_pages_fp8": (
        c_int,
        [c_void_p, c_int, c_int, c_int, c_int, c_int, c_int, c_void_p, c_int64, c_void_p, c_void_p, c_void_p, c_void_p],
    ),
    "fs_dequantize_fp8": (c_int, [c_void_p, c_void_p, c_int64, c_int, c_int, c_int, c_int, c_void_p, c_int, c_void_p]),
    "fs_fused_decode_fp8": (
        c_int,
        [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_int, c_int,
         c_int, c_int, c_int, c_int, c_float, c_int, c_int, c_int, c_void_p],
    ),
    "fs_paged_decode_fp8": (
        c_int,
        [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int64, c_void_p, c_void_p,
         c_void_p, c_int64, c_int, c_int, c_int, c_int64, c_int, c_int, c_int, c_float, c_int, c_int, c_int, c_void_p],
    ),
    "fs_combine_splits": (
        c_int, [c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int, c_int, c_int, c_void_p]
    ),
    "fs_quantize_i8": (
        c_int, [c_void_p, c_int, c_int64, c_int, c_int, c_int, c_void_p, c_void_p, c_void_p, c_void_p]
    ),
    "fs_dequantize_i8": (
        c_int, [c_void_p, c_void_p, c_void_p, c_int64, c_int, c_int, c_int, c_int, c_void_p, c_int, c_void_p]
    ),
    "fs_quantize_pages_i8": (
        c_int,
        [c_void_p, c_int, c_int, c_int, c_int, c_int, c_int, c_void_p, c_int64, c_void_p, c_void_p, c_void_p,
         c_void_p],
    ),
    "fs_update_pages_i8": (
        c_int,
        [c_void_p, c_void_p, c_void_p, c_int64, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int64,
         c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int, c_void_p],
    ),
    "fs_quantize_sym_i8": (
        c_int, [c_void_p, c_int, c_int64, c_int, c_void_p, c_void_p, c_void_p, c_void_p]
    ),
    "fs_append_tokens_i8": (
        c_int,
        [c_void_p, c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_void_p,
         c_int, c_int, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_void_p, c_void_p],
    ),
    "fs_paged_decode_ordered": (
        c_int,
        [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int64,
         c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_int64, c_int, c_int, c_int, c_int64, c_int,
         c_int, c_int, c_float, c_int, c_int, c_int, c_void_p],
    ),
    "fs_paged_decode_append_i8": (
        c_int,
        [c_void_p, c_int, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
         c_int, c_int64, c_void_p, c_void_p, c_void_p, c_void_p, c_int64, c_void_p, c_int64, c_int, c_int, c_int,
         c_int64, c_int, c_int, c_float, c_int, c_int, c_int, c_void_p, c_void_p],
    ),
}

_lib = None
LOAD_ERROR: str | None = None


def _load() -> None:
    global _lib, LOAD_ERROR
    try:
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        LOAD_ERROR = None
    except (OSError, AttributeError) as exc:  # missing/stale .so
        _lib = None
        LOAD_ERROR = f"{type(exc).__name__}: {exc}"


_load()


def available() -> bool:
    return _lib is not None


def require():
    if _lib is None:
        raise RuntimeError(
            f"libflashspec_hip.so is not loaded ({LOAD_ERROR}); build it with "
            "`python -m flashspec_amd._build` — GPU tensors have no other implementation"
        )
    return _lib


def reload() -> bool:
    """Retry opening the library (e.g. after building it in this process).

    A library already opened by this process is not re-read from disk: rebuild
    before starting the process that uses it.
    """

    _load()
    return available()


def check(rc: int) -> None:
    """Map a C status to the reference's exception classes."""

    if rc == FS_OK:
        return
    msg = _lib.fs_last_error().decode(errors="replace") if _lib is not None else "unknown error"
    if rc == FS_ERR_INVALID:
        raise ValueError(msg)
    raise RuntimeError(msg)


def ptr(t: torch.Tensor | None):
    return None if t is None else t.data_ptr()


def dtype_code(dtype: torch.dtype) -> int:
    try:
        return DTYPE_CODE[dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {dtype}; expected float16, bfloat16 or float32") from None


# torch's raw current-stream query (the handle alone, without building a Stream object: ~0.2 instead
# of ~2 us per launch); torch.cuda.current_stream where a build lacks it.
_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_ptr(device: torch.device) -> int:
    """hipStream_t of the current stream on ``device``, as an integer."""

    if _RAW_STREAM is not None:
        return _RAW_STREAM(device.index if device.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(device).cuda_stream
