"""The quantizer kernel (csrc/quant_kernels.hip, quantize_row) replaces the
per-element division X / s of the reference's quantizers
(tests/test_kernels.py:32-34, nb:292-299) by one reciprocal per row and a
Markstein correction step. These CPU checks compile tests/quant_divide_check.c
with gcc and compare that arithmetic with the IEEE division: every finite fp16
x against a spread of fp16 scales (the full product of both, about 2e9 pairs,
was checked once as well), and random fp32 pairs with quotients at and next to
the rounding ties."""

import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))

pytestmark = pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    exe = str(tmp_path_factory.mktemp("qdiv") / "quant_divide_check")
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", os.path.join(HERE, "quant_divide_check.c"),
                    "-o", exe, "-lm"], check=True)
    return exe


def run(exe, *args):
    res = subprocess.run([exe] + [str(a) for a in args], stdout=subprocess.PIPE, text=True, timeout=300)
    assert res.returncode == 0, res.stdout
    return res.stdout


def test_fp16_values_against_fp16_scales(checker):
    out = run(checker, "fp16", 61)  # every 61st scale: all exponents, ~32M pairs
    assert "mismatches 0" in out


def test_fp32_random_and_near_ties(checker):
    out = run(checker, "fp32", 5_000_000)
    assert "mismatches 0" in out
