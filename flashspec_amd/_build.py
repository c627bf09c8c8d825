"""Build libflashspec_hip.so in-tree with hipcc for gfx950.

``python -m flashspec_amd._build [--resource-usage]`` compiles every ``csrc/*.hip``
to an object under ``_build/`` (in parallel) and links the shared library next to
this file, where ``flashspec_amd._lib`` loads it.  No torch headers are used.
"""

from __future__ import annotations

import argparse
import json
import os
import re
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
BUILD = PKG.parent / "_build"
LIB_NAME = "libflashspec_hip.so"
ARCH = os.environ.get("FLASHSPEC_OFFLOAD_ARCH", "gfx950")

# Packed-FP32 instructions stay disabled (see csrc/fs_common.h users); the host pass
# warns that it does not know the feature, which is harmless.
COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-result",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found; set HIPCC")


# Per-source flags.  The tiled decode kernel leads its arguments with seven 64-bit start-up words
# that gfx950 preloads into SGPRs (kernel-argument preload, 14 dwords).
SOURCE_FLAGS = {
    "fs_decode.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=7"],
}


def _compile(src: Path, extra: list[str]) -> tuple[Path, str]:
    obj = BUILD / (src.stem + ".o")
    cmd = [hipcc(), *COMMON_FLAGS, *SOURCE_FLAGS.get(src.name, []), *extra, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stderr[-8000:]}")
    lines = [ln for ln in proc.stderr.splitlines() if ("warning" in ln or "error" in ln)
             and "packed-fp32-ops" not in ln]
    if lines:
        sys.stderr.write("\n".join(lines) + "\n")
    return obj, proc.stderr


RESOURCES = PKG / "kernel_resources.json"
_REMARK = re.compile(r"remark:\s+(Function Name|VGPRs|AGPRs|TotalSGPRs|ScratchSize \[bytes/lane\]|"
                     r"Occupancy \[waves/SIMD\]|LDS Size \[bytes/block\]):\s+(\S+)")


def _parse_resources(text: str) -> list[dict]:
    """Per-kernel VGPR/SGPR/LDS/occupancy from clang's kernel-resource-usage remarks."""

    kernels, cur = [], None
    for m in _REMARK.finditer(text):
        key, val = m.group(1), m.group(2)
        if key == "Function Name":
            cur = {"kernel": val}
            kernels.append(cur)
        elif cur is not None:
            cur[key.split(" [")[0].lower()] = int(val) if val.isdigit() else val
    return kernels


def build(resource_usage: bool = True, jobs: int = 4) -> Path:
    """Compile and link; returns the path of the shared library.

    With ``resource_usage`` the per-kernel register/LDS/occupancy table of the device
    code is written to ``kernel_resources.json`` beside the library.
    """

    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    extra = ["-Rpass-analysis=kernel-resource-usage"] if resource_usage else []
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as pool:
        results = list(pool.map(lambda s: _compile(s, extra), sources))
    objs = [o for o, _ in results]
    if resource_usage:
        table = [k for _, text in results for k in _parse_resources(text)]
        RESOURCES.write_text(json.dumps({"arch": ARCH, "kernels": table}, indent=1) + "\n")
    lib = PKG / LIB_NAME
    tmp = PKG / (LIB_NAME + ".tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr[-8000:]}")
    os.replace(tmp, lib)
    return lib


def _demangle(names: list[str]) -> list[str]:
    tool = shutil.which("llvm-cxxfilt") or shutil.which("c++filt") or "c++filt"
    try:
        out = subprocess.run([tool], input="\n".join(names), capture_output=True, text=True, check=True).stdout
        return out.splitlines()
    except (OSError, subprocess.CalledProcessError):
        return names


def resources_markdown() -> str:
    """The register/LDS/occupancy table of ``kernel_resources.json`` as Markdown."""

    data = json.loads(RESOURCES.read_text())
    kernels = data["kernels"]
    names = _demangle([k["kernel"] for k in kernels])
    lines = [f"| kernel ({data['arch']}) | VGPRs | AGPRs | SGPRs | scratch B/lane | LDS B/block | waves/SIMD |",
             "|---|---:|---:|---:|---:|---:|---:|"]
    for k, name in zip(kernels, names):
        lines.append(f"| `{name.replace('fs::DecodeParams', 'DecodeParams')}` | {k.get('vgprs')} | {k.get('agprs')} | "
                     f"{k.get('totalsgprs')} | {k.get('scratchsize')} | {k.get('lds size')} | {k.get('occupancy')} |")
    return "\n".join(lines) + "\n"


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--no-resource-usage", action="store_true", help="skip the register/occupancy table")
    ap.add_argument("--print-resources", action="store_true", help="print the last table as Markdown and exit")
    ap.add_argument("-j", "--jobs", type=int, default=4)
    args = ap.parse_args()
    if args.print_resources:
        print(resources_markdown(), end="")
        return
    print(build(resource_usage=not args.no_resource_usage, jobs=args.jobs))


if __name__ == "__main__":
    main()
