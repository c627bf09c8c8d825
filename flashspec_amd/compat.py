"""Make ``import flashspec`` (and its submodules) resolve to this package.

    import flashspec_amd.compat  # noqa: F401  -- once, before importing flashspec
    from flashspec import paged_quant_attention_triton
    import flashspec.triton_fused as triton_fused

Existing reference call sites then run unchanged on the HIP backend.  Refuses to
shadow a different ``flashspec`` that is already imported.
"""

from __future__ import annotations

import sys

import flashspec_amd
from flashspec_amd import attention, paged, quant, runtime, serving, tree, triton_fused, triton_paged, triton_utils

_SUBMODULES = {
    "attention": attention,
    "paged": paged,
    "quant": quant,
    "runtime": runtime,
    "serving": serving,
    "tree": tree,
    "triton_fused": triton_fused,
    "triton_paged": triton_paged,
    "triton_utils": triton_utils,
}


def install() -> None:
    existing = sys.modules.get("flashspec")
    if existing is not None and existing is not flashspec_amd:
        raise ImportError("a different 'flashspec' package is already imported")
    sys.modules["flashspec"] = flashspec_amd
    for name, mod in _SUBMODULES.items():
        sys.modules[f"flashspec.{name}"] = mod


install()
