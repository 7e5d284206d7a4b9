"""The A8 prologue's fast quotient (reciprocal + one residual correction) against the IEEE
division, over every pair of 16-bit values the quantizer can see (tests/quotient_check.c).

fp16: the fp32 quotients are identical.  bf16: the int8 results are identical; the fp32 quotient
differs for x so small (|x| near 2^-126 or below) that the residual x - q0 s is an fp32 subnormal
and inexact, and every such quotient quantizes to the same int8.  CPU only: compiled with gcc,
no GPU."""
import re
import shutil
import subprocess

import pytest

HERE = __import__("os").path.dirname(__file__)


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    exe = tmp_path_factory.mktemp("qc") / "quotient_check"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", str(exe), f"{HERE}/quotient_check.c", "-lm", "-lpthread"],
                   check=True)
    return str(exe)


def run(exe, fmt):
    out = subprocess.run([exe, fmt], check=True, capture_output=True, text=True, timeout=300).stdout
    m = re.search(r"pairs=(\d+) f32_mismatch=(\d+) int8_mismatch=(\d+)", out)
    assert m, out
    return tuple(int(g) for g in m.groups())


def test_fp16_quotient_exact(checker):
    pairs, f32_bad, int8_bad = run(checker, "h")
    assert pairs > 10 ** 8
    assert f32_bad == 0 and int8_bad == 0


def test_bf16_quantized_exact(checker):
    pairs, f32_bad, int8_bad = run(checker, "b")
    assert pairs > 10 ** 8
    assert int8_bad == 0
