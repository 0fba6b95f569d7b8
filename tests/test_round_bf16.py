"""The product's bf16 rounding (the shared host/device numerics header every kernel inlines) equals
the oracle's on all 2^32 f32 bit patterns. The oracle's rounding is pinned by the reference's
bf16-boundary golden vectors; the GPU side of the header is held to the oracle by the bit-exact
kernel tests."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
ORACLE = os.path.join(ROOT, "oracle")
CSRC = os.path.join(ROOT, "mimo-prismwing_amd", "csrc")


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_round_bf16_equals_oracle_exhaustively(tmp_path):
    exe = str(tmp_path / "round_bf16_check")
    base = ["g++", "-O2", "-std=c++20", "-I" + CSRC, os.path.join(HERE, "round_bf16_check.cpp"), "-o", exe,
            "-L" + ORACLE, "-lpw_oracle", "-Wl,-rpath," + ORACLE]
    # OpenMP where the compiler has it (about 10 s of work on one core)
    if subprocess.run(base[:1] + ["-fopenmp"] + base[1:], capture_output=True).returncode != 0:
        subprocess.run(base, check=True, capture_output=True)
    out = subprocess.run([exe], capture_output=True, text=True, timeout=600)
    assert out.returncode == 0, out.stdout
    assert out.stdout.split() == ["inputs", "4294967296", "mismatches", "0"], out.stdout
