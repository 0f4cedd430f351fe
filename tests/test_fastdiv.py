"""The multiply-shift division of csrc/fa_fastdiv.h (used for the block
descriptors of the persistent kernels), compiled for the host with g++ from
the same header and checked against hardware division over every dividend
below 2^18 for every divisor below 2^12 and near the 2^31 bounds."""
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not available")
def test_fastdiv_matches_division(tmp_path):
    exe = tmp_path / "fastdiv_check"
    subprocess.run(["g++", "-O2", "-std=c++17", f"-I{ROOT / 'flash-attn-triton_amd' / 'csrc'}",
                    str(ROOT / "tests" / "fastdiv_check.cpp"), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "wrong 0" in out.stdout
