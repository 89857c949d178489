"""The kernels' temperature division (``div_rt`` in csrc/fl_device.h: one
reciprocal per row, then Markstein's FMA correction) equals IEEE float32
division bit for bit (CPU only; the C checker uses the host's fmaf).

By default: every bfloat16 value against 2000 divisors, and against 1500
divisors spread over the whole float range (2^-127 .. 2^127, where
``recip_rt`` sends the ones outside [2^-100, 2^100] to the division itself),
and every 97th float32 value against 2 divisors (~12 s).  FL_FULL_DIVISION_SWEEP=1 runs every
bfloat16 value against 200000 divisors and every finite float32 value against
8 divisors (~3 min)."""

import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


def test_markstein_division_equals_ieee_division(tmp_path):
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    exe = str(tmp_path / "division_check")
    # -ffp-contract=off: x * rt is its own rounded product, as on the GPU
    subprocess.run([gcc, "-O2", "-ffp-contract=off", os.path.join(HERE, "division_check.c"), "-o", exe, "-lm"],
                   check=True)
    args = ["200000", "1", "8"] if os.environ.get("FL_FULL_DIVISION_SWEEP") == "1" else ["2000", "97", "2"]
    res = subprocess.run([exe, *args], capture_output=True, text=True)
    lines = dict((ln.split()[0], ln.split()[1:]) for ln in res.stdout.strip().splitlines() if not ln.startswith("bad"))
    assert res.returncode == 0, res.stdout[-2000:]
    assert int(lines["bf16"][0]) > 100_000_000 and int(lines["bf16"][1]) == 0
    assert int(lines["f32"][0]) > 80_000_000 and int(lines["f32"][1]) == 0
    assert int(lines["wide"][0]) > 90_000_000 and int(lines["wide"][1]) == 0
