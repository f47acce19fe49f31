"""The append kernels divide with a per-row reciprocal and two FMAs
(rtn_i8_recip in s8kv_device.h for the int8 codes, the block-norm quotient
of rows_lloydmax3_store in s8kv_append.hip for K8V3).  Their bytes equal the
oracle's only if those quotients are the IEEE quotients.  The C checkers beside
this test compare the two: for int8 on every (y, absmax) pair the kernel can
meet (y fp16, scale = absmax / 127 for an fp16 absmax >= |y|), about 1.0e9
pairs, with the kernel's clamp-free rounding of the quotient; for K8V3 on
every pair of an fp16 significand and an fp32 norm significand (8.6e9 pairs,
which stand for all operands by exact power-of-two scaling) plus a sample over
the whole domain.  Both run with the CPU's fmaf; each was seen to fail when
the correcting FMA is dropped."""

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


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_norm_quotient_equals_ieee_quotient(tmp_path):
    exe = tmp_path / "lloyd_quotient_check"
    cmd = ["gcc", "-O2", "-ffp-contract=off", "-o", str(exe), os.path.join(HERE, "lloyd_quotient_check.c"), "-lm"]
    if "fma" in open("/proc/cpuinfo").read():
        cmd.insert(2, "-mfma")
    omp = subprocess.run(cmd[:1] + ["-fopenmp", "-x", "c", "-", "-o", os.devnull], input="int main(void){return 0;}",
                         capture_output=True, text=True)
    if omp.returncode == 0:
        cmd.insert(2, "-fopenmp")
    subprocess.run(cmd, check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600)
    last = out.stdout.strip().splitlines()[-1]
    assert out.returncode == 0 and last.endswith("mismatches 0"), out.stdout
    assert int(last.split()[1]) > 8_589_934_592
