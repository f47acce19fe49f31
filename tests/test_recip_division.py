"""The append kernel quantizes with rint(y / scale) computed from a per-row
reciprocal and two FMAs (rtn_i8_recip in s8kv_device.h).  Its bytes equal the
oracle's only if that quotient is the IEEE quotient; the C checker beside this
test compares the two on every (y, absmax) pair the kernel can meet (y fp16,
scale = absmax / 127 for an fp16 absmax >= |y|), about 1.0e9 pairs, with the
CPU's fmaf."""

import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_reciprocal_quotient_equals_ieee_quotient(tmp_path):
    exe = tmp_path / "recip_division_check"
    subprocess.run(["gcc", "-O2", "-ffp-contract=off", "-o", str(exe), os.path.join(HERE, "recip_division_check.c"),
                    "-lm"], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    last = out.stdout.strip().splitlines()[-1]
    assert out.returncode == 0 and last.endswith("mismatches 0"), out.stdout
    assert int(last.split()[1]) > 1_000_000_000
