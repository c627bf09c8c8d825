"""Device / dtype helpers with the reference's semantics (src/flashspec/runtime.py:6-109)."""

from __future__ import annotations

import torch


def resolve_device(device: str = "auto") -> torch.device:
    """``auto`` -> cuda when available (ROCm devices report type "cuda"), else cpu.

    An explicit cuda request without a GPU raises RuntimeError (runtime.py:25-34).
    """

    if device == "auto":
        return torch.device("cuda" if torch.cuda.is_available() else "cpu")
    resolved = torch.device(device)
    if resolved.type == "cuda" and not torch.cuda.is_available():
        raise RuntimeError("cuda was requested but torch.cuda.is_available() is false")
    return resolved


_DTYPES = {
    "float16": torch.float16,
    "fp16": torch.float16,
    "bfloat16": torch.bfloat16,
    "bf16": torch.bfloat16,
    "float32": torch.float32,
    "fp32": torch.float32,
}


def resolve_dtype(dtype: str = "auto", device: torch.device | None = None) -> torch.dtype:
    """``auto`` -> float16 on GPU, float32 on CPU (runtime.py:37-73)."""

    if dtype == "auto":
        return torch.float16 if device is not None and device.type == "cuda" else torch.float32
    if dtype not in _DTYPES:
        raise ValueError(f"unsupported dtype: {dtype}")
    return _DTYPES[dtype]


def synchronize(device: torch.device) -> None:
    if device.type == "cuda":
        torch.cuda.synchronize(device)


def device_name(device: torch.device) -> str:
    if device.type == "cuda":
        return torch.cuda.get_device_name(device)
    return "cpu"
