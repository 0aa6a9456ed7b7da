"""The device requantization's fast paths (``qa_mbqm_fast`` in
``qa_common.h``: an int64 product for |x| < 2^32, two 32x32-bit products for
|x| < 2^62) against the plain 128-bit form, compiled for the host."""

import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HIPCC = "/opt/rocm/bin/hipcc"


@pytest.mark.skipif(shutil.which(HIPCC) is None, reason="no hipcc")
def test_mbqm_fast_paths_equal_128_bit_form(tmp_path):
    exe = tmp_path / "mbqm_paths"
    subprocess.run([HIPCC, "-O2", "-std=c++17",
                    f"-I{ROOT / 'quantanything_amd' / 'csrc'}",
                    str(ROOT / "tests" / "native" / "mbqm_paths.cpp"),
                    "-o", str(exe)], check=True, capture_output=True)
    out = subprocess.run([str(exe), "2000000"], capture_output=True,
                         text=True)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "mismatches 0" in out.stdout
