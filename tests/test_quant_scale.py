"""The bf16 quantisers' scale without a division (the shared host/device numerics header every
kernel inlines) equals the oracle quantiser's max(m, 1e-10) / 448 for every non-negative finite
bf16 group maximum m. The oracle's quantiser is pinned by the reference's dynamic-FP8 golden
vector; the GPU side of the header is held to the oracle by the quantiser sweeps and the bit-exact
prefill tests."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
ORACLE = os.path.join(ROOT, "oracle")
CSRC = os.path.join(ROOT, "mimo-prismwing_amd", "csrc")


@pytest.mark.skipif(shutil.which("g++") is None, reason="needs g++")
def test_scale_of_bf16_max_equals_oracle_exhaustively(tmp_path):
    exe = str(tmp_path / "quant_scale_check")
    subprocess.run(["g++", "-O2", "-std=c++20", "-ffp-contract=off", "-I" + CSRC,
                    os.path.join(HERE, "quant_scale_check.cpp"), "-o", exe, "-L" + ORACLE, "-lpw_oracle",
                    "-Wl,-rpath," + ORACLE], check=True, capture_output=True)
    out = subprocess.run([exe], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stdout
    assert out.stdout.split() == ["maxima", "32640", "mismatches", "0"], out.stdout
