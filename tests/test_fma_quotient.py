"""The KIVI quantiser (halo_amd/csrc/kivi.hip, kivi_code_fma) forms the
quotient (x - zero) / scale as q = d * (1/s) plus one FMA correction
instead of a division.  This runs the exhaustive host check
(tests/native/fma_quotient_check.c): for every pair of fp16 values, and
every pair of bf16 values inside [2^-63, 2^63], the corrected product equals
the IEEE fp32 quotient bit for bit (the kernel divides outside that range).
CPU only; needs gcc."""
from __future__ import annotations

import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.parametrize("fmt", ["fp16", "bf16"])
def test_fma_corrected_quotient_equals_division(tmp_path, fmt):
    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    exe = tmp_path / "check"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", str(exe),
                    os.path.join(HERE, "native", "fma_quotient_check.c"), "-lm"], check=True)
    r = subprocess.run([str(exe), fmt], capture_output=True, text=True, timeout=600)
    assert r.returncode == 0, r.stdout
    assert " 0 differ" in r.stdout
