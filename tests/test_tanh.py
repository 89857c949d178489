"""The kernels' soft-cap tanh (``fl_tanh`` in csrc/fl_device.h: an odd
polynomial below |z| = 0.625, tanhf above) against double-precision tanh
(CPU only; the C checker uses the host's fmaf, which rounds as the GPU's FMA
does).  Over every float32 value in [0, 0.625) it must lie within 0.75 ulp of
tanh, equal the correctly rounded value for all but 0.1 % of the values, and
never decrease (the two-read float32 path bins values by a monotone order):
each checked value is compared with the polynomial at the next float up, and
the constant that floors the tanhf branch above 0.625 must be the
polynomial's value at the largest float below it.

By default every 5th float32 value (~15 s); FL_FULL_TANH_SWEEP=1 checks every
value (~70 s)."""

import os
import re
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
DEVICE_H = os.path.join(HERE, "..", "rl_project_amd", "csrc", "fl_device.h")


def _coefficients():
    text = open(DEVICE_H).read()
    m = re.search(r"constexpr float TANH_P\[6\] = \{([^}]*)\};", text)
    assert m, "TANH_P not found in fl_device.h"
    vals = [v.strip().rstrip("f") for v in m.group(1).split(",")]
    assert len(vals) == 6
    return vals


def test_polynomial_tanh_within_an_ulp_and_monotone(tmp_path):
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not available")
    exe = str(tmp_path / "tanh_check")
    # -ffp-contract=off: z * z and z * t are rounded products, as on the GPU
    subprocess.run([gcc, "-O2", "-ffp-contract=off", os.path.join(HERE, "tanh_check.c"), "-o", exe, "-lm"],
                   check=True)
    stride = 1 if os.environ.get("FL_FULL_TANH_SWEEP") == "1" else 5
    res = subprocess.run([exe, str(stride), *_coefficients()], capture_output=True, text=True, timeout=600)
    assert res.returncode == 0, res.stdout + res.stderr
    f = res.stdout.split()
    checked, differ, max_err, decreases = int(f[1]), int(f[3]), float(f[5]), int(f[7])
    assert checked > 1_000_000_000 // stride
    assert max_err <= 0.75
    assert differ <= checked // 1000
    assert decreases == 0
    # the floor of the tanhf branch is the polynomial's last value below the switch
    m = re.search(r"constexpr uint32_t TANH_AT_SWITCH_BITS = (0x[0-9a-fA-F]+)u;", open(DEVICE_H).read())
    assert m and int(m.group(1), 16) == int(f[9], 16), (f[9], m and m.group(1))
