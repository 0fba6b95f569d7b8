"""The bf16 quantisers' division (one correctly rounded reciprocal per group, then a Markstein-
corrected quotient per value) gives the same e4m3fn codes as the IEEE quotient for every bf16
value against every bf16 group absmax (1,065,402,238 pairs). The check is plain C over IEEE f32
arithmetic with explicit fused multiply-adds, the same operations the device code issues; the GPU
side is held to the oracle by test_quantiser_bf16_division_sweep."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE = os.path.join(os.path.dirname(HERE), "oracle")


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_quant_ratio_codes_equal_ieee_division_exhaustively(tmp_path):
    exe = str(tmp_path / "quant_ratio_check")
    base = ["gcc", "-O2", "-std=c11", "-ffp-contract=off", "-fno-fast-math",
            os.path.join(HERE, "quant_ratio_check.c"), "-o", exe, "-L" + ORACLE, "-lpw_oracle",
            "-Wl,-rpath," + ORACLE, "-lm"]
    # OpenMP where the compiler has it (about 50 s of work on one core)
    if subprocess.run(base[:1] + ["-fopenmp"] + base[1:], capture_output=True).returncode != 0:
        subprocess.run(base, check=True, capture_output=True)
    out = subprocess.run([exe], capture_output=True, text=True, timeout=600)
    assert out.returncode == 0, out.stdout
    assert out.stdout.split()[:4] == ["pairs", "1065402238", "code_mismatches", "0"], out.stdout
