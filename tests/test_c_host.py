"""The C ABI from a plain C99 host (CPU): tests/c_host/abi_check.c includes
include/flashspec_hip.h, links flashspec_amd/libflashspec_hip.so with gcc and makes the calls
that need no GPU — the header is valid C and the library resolves from a non-Python host."""

from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

from flashspec_amd import _lib

ROOT = Path(__file__).resolve().parents[1]


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_c99_host_links_and_calls_the_abi(tmp_path):
    assert _lib.available(), _lib.LOAD_ERROR
    lib = Path(_lib.LIB_PATH).resolve()
    exe = tmp_path / "abi_check"
    subprocess.run(["gcc", "-std=c99", "-Wall", "-Werror", "-I", str(ROOT / "include"),
                    str(ROOT / "tests" / "c_host" / "abi_check.c"), "-o", str(exe), str(lib),
                    f"-Wl,-rpath,{lib.parent}"], check=True)
    proc = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert proc.returncode == 0, proc.stdout + proc.stderr
    assert proc.stdout.count("ok ") == 6, proc.stdout
