"""Shared test setup.

Tests marked `gpu` need an MI355X and the built lib/libgaje_hip.so; everything
else runs on the CPU (oracle against the reference's known answers, the reader,
host logic, and the C-ABI symbol table).
"""
import os
import sys

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "gaje-semantic-compression_amd")
for p in (REPO, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


def floored_rel_err(got, ref) -> float:
    """max_i |got_i - ref_i| / max(|ref_i|, tau) with tau = 1e-3 * max|ref|.

    A plain elementwise relative error is ill-posed for these outputs: the
    reference flushes |t| < 1e-6 to 0 and summation-order noise dominates near
    zero, so the denominator is floored at a thousandth of the largest output.
    """
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    if ref.size == 0:
        return 0.0
    tau = 1e-3 * float(np.max(np.abs(ref)))
    den = np.maximum(np.abs(ref), tau)
    den[den == 0] = 1.0
    return float(np.max(np.abs(got - ref) / den))


@pytest.fixture(scope="session")
def tmp_models(tmp_path_factory):
    """Directory for synthetic .gaje.flat files written during the session."""
    return tmp_path_factory.mktemp("models")
