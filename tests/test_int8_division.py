"""The INT8 Q quantizer replaces the IEEE division x / s by a reciprocal and
one Markstein correction (quant_div, flash-attn-triton_amd/csrc/fa_int8.h).
The quantized values must stay bit-exact with the reference's division form
(attention_kernel_int8.py:100), so the replacement is checked exhaustively
over its whole input domain on the CPU: every fp16 amax, every fp16 x with
|x| <= amax (7.7e8 pairs), compiled with gcc and correctly rounded fmaf.
A mistake in the correction step (a dropped remainder term, a wrong sign)
fails at once; the GPU's v_fma_f32 is IEEE fused multiply-add like fmaf.
"""
import shutil
import subprocess
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_markstein_quotient_equals_ieee_division(tmp_path):
    exe = tmp_path / "int8_division_check"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", str(HERE / "int8_division_check.c"),
                    "-o", str(exe), "-lm"], check=True)
    out = subprocess.run([str(exe)], check=True, capture_output=True, text=True, timeout=300)
    pairs, bad = (int(x) for x in out.stdout.split())
    assert pairs > 7.7e8
    assert bad == 0
