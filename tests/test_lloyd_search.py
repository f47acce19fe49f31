"""The K8V3 append picks each value's codeword with three comparisons (a binary
search over "entry j is strictly nearer than entry j - 1", lloyd3_search in
s8kv_device.h; the rows kernel of s8kv_append.hip compares u against
per-codebook thresholds T_j, the least u where that test holds, found by
bisection) where the oracle scans all eight entries for the first minimum.
They agree for codebooks that pass lloyd3_search_ok (ascending, within
[-4, 4], neighbours at least 2^-19 apart) and |u| <= 1.  The C checker beside
this test compares both forms with the scan on every fp32 u in [-1, 1] and
NaN, for the package codebook, a codebook at the smallest allowed spacing, one
reaching +-4 and random ones; it reports mismatches when T_4 is moved one
fp32 step down, and rejects a codebook outside the condition."""

import os
import shutil
import subprocess

import numpy as np
import pytest

from superl8_serve_amd.codebook import gaussian_codebook

HERE = os.path.dirname(os.path.abspath(__file__))


def _codebooks():
    rng = np.random.default_rng(11)
    books = [gaussian_codebook(),
             np.array([(j - 3) * 2.0 ** -19 for j in range(8)], dtype=np.float32),
             np.array([-4.0, -1.5, -0.25, -2.0 ** -19, 0.0, 0.3, 1.0, 4.0], dtype=np.float32)]
    for _ in range(2):
        books.append(np.sort(rng.uniform(-1.2, 1.2, 8)).astype(np.float32))
    return books


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    if shutil.which("gcc") is None:
        pytest.skip("needs gcc")
    exe = tmp_path_factory.mktemp("lloyd") / "lloyd_search_check"
    cmd = ["gcc", "-O2", "-ffp-contract=off", "-o", str(exe), os.path.join(HERE, "lloyd_search_check.c"), "-lm"]
    omp = subprocess.run(["gcc", "-fopenmp", "-x", "c", "-", "-o", os.devnull], input="int main(void){return 0;}",
                         capture_output=True, text=True)
    if omp.returncode == 0:
        cmd.insert(2, "-fopenmp")
    subprocess.run(cmd, check=True)
    return exe


@pytest.mark.parametrize("idx", range(5))
def test_search_equals_first_minimum_scan(checker, idx):
    cb = _codebooks()[idx]
    assert np.all(np.diff(cb) >= 2.0 ** -19)
    out = subprocess.run([str(checker), *[float(c).hex() for c in cb]], capture_output=True, text=True, timeout=300)
    last = out.stdout.strip().splitlines()[-1]
    assert out.returncode == 0 and last.endswith("mismatches 0"), out.stdout
    assert int(last.split()[1]) == 2 * 0x3F800001 + 1


def test_codebook_outside_condition_rejected(checker):
    for cb in ([0, 1, 2, 3, 4, 5, 6, 7], [0.0, 0.1, 0.2, 0.3, 0.3, 0.5, 0.6, 0.7]):
        out = subprocess.run([str(checker), *map(str, cb)], capture_output=True, text=True, timeout=60)
        assert out.returncode == 2 and out.stdout.strip() == "rejected"


def test_threshold_one_step_low_reported(checker):
    cb = gaussian_codebook()
    out = subprocess.run([str(checker), *[float(c).hex() for c in cb], "lower"], capture_output=True, text=True,
                         timeout=300)
    last = out.stdout.strip().splitlines()[-1]
    assert out.returncode == 1 and int(last.split()[-1]) >= 1, out.stdout
