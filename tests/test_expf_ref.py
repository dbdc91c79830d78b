"""The device exponential restates the C library expf that the reference's
f32::exp calls (attention.rs:106, activation.rs:42-44) bit for bit.

Compiles csrc/expf_ref.h for the host and compares it with the host libm over
every single-precision input (about 15 s on 8 cores).  This pins the
restatement; tests/test_gpu_ops.py then pins the device build against it.
"""
import os
import subprocess

import pytest

from conftest import PKG, REPO


@pytest.fixture(scope="module")
def sweep_bin(tmp_path_factory):
    out = str(tmp_path_factory.mktemp("expf") / "expf_sweep")
    subprocess.run(["g++", "-O2", "-ffp-contract=off", "-fopenmp", "-std=c++17",
                    "-I", os.path.join(PKG, "csrc"), os.path.join(REPO, "tests", "expf_sweep.cpp"),
                    "-o", out, "-lm"], check=True)
    return out


def test_expf_ref_matches_libm_on_all_floats(sweep_bin):
    r = subprocess.run([sweep_bin, "1"], check=True, capture_output=True, text=True, timeout=600)
    mism, n = map(int, r.stdout.split())
    assert n == 2 ** 32
    assert mism == 0, f"{mism} of {n} inputs differ from the host expf"
