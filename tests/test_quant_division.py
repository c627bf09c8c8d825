"""The vectorized quantizer divides by the block scale with a reciprocal and one FMA
correction step (flashspec_amd/csrc/fs_common.h, div_by_scale).  This checks, on the CPU
with a correctly rounded fmaf, that the step reproduces IEEE float32 division bit for bit
over every finite fp16 input and random fp32 inputs, for quantizer-like scales, all-ones
significands and random normal scales (only the sign of a zero quotient may differ)."""

from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

SRC = Path(__file__).resolve().parent / "cdiv" / "markstein_check.c"


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_reciprocal_fma_division_matches_ieee(tmp_path):
    exe = tmp_path / "markstein_check"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", str(exe), str(SRC), "-lm"], check=True)
    proc = subprocess.run([str(exe), "600", "20000"], capture_output=True, text=True, timeout=300)
    assert proc.returncode == 0, proc.stdout[-2000:]
    total, bad = (int(w) for w in proc.stdout.split()[-3::2])
    assert bad == 0 and total > 40_000_000
