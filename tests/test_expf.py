"""The GPU router's exp (anedvd_amd/csrc/expf_exact.h) equals the host libm expf on
every float input, so device routing reproduces the CPU's softmax bit for bit."""
import os
import subprocess
import tempfile

import pytest

from tests.conftest import ROOT


@pytest.mark.slow
def test_expf_exact_matches_libm_on_all_floats():
    with tempfile.TemporaryDirectory() as td:
        exe = os.path.join(td, "expf_exhaustive")
        subprocess.run(["g++", "-O2", "-fopenmp", "-ffp-contract=off", "-std=c++17",
                        "-I", os.path.join(ROOT, "anedvd_amd", "csrc"),
                        os.path.join(ROOT, "tests", "expf_exhaustive.cpp"), "-o", exe, "-lm"], check=True)
        r = subprocess.run([exe], capture_output=True, text=True, timeout=600)
        assert r.returncode == 0, r.stdout + r.stderr
        assert "mismatches 0" in r.stdout
