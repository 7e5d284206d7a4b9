"""The A8 weight decoders' int8 grid arithmetic (a rounding add of 1.5 * 2^23, a float clamp and the
low byte of the bit pattern) against clamp(rne(fp32(level * s)), -127, 127), the reference's
definition (modal/weight_error_app.py:335-337), over every 4- and 6-bit code and every fp16, bf16
and e4m3 scale, 2^24 random fp32 scales and the fixed codebook (tests/grid_decode_check.c).
CPU only: compiled with gcc, no GPU."""
import os
import re
import shutil
import subprocess

import pytest

HERE = os.path.dirname(__file__)


def test_grid_decode_matches_the_reference_definition(tmp_path):
    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    exe = tmp_path / "grid_decode_check"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", str(exe), f"{HERE}/grid_decode_check.c", "-lm"],
                   check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300).stdout
    m = re.search(r"checked=(\d+) mismatch=(\d+)", out)
    assert m, out
    assert int(m.group(1)) > 1_000_000_000 and int(m.group(2)) == 0, out
