"""Exhaustive CPU check of the quantizer's reciprocal-based division (div_by_scale in
csrc/fp8_common.h): over every (amax, element) pair of bf16 and of fp16 it gives the bits
of IEEE division wherever they can reach an e4m3 code (tests/c/quant_division_check.c).
The GPU quantizer is then held to the oracle's IEEE division by the GPU parity tests."""

import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    exe = str(tmp_path_factory.mktemp("divcheck") / "quant_division_check")
    subprocess.run([gcc, "-O2", "-ffp-contract=off", "-fopenmp", "-o", exe,
                    os.path.join(HERE, "c", "quant_division_check.c"), "-lm"], check=True)
    return exe


@pytest.mark.parametrize("fmt", ["b", "h"])
def test_division_matches_ieee_exhaustively(checker, fmt):
    run = subprocess.run([checker, fmt], capture_output=True, text=True, timeout=600)
    assert run.returncode == 0, run.stdout + run.stderr
    assert " 0 mismatches" in run.stdout
