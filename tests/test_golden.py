"""The oracle still reproduces the committed golden fixtures bit for bit
(tests/golden/make_golden.py wrote them; the GPU suite checks the HIP path
against the same files)."""
import hashlib
import os
import sys

import numpy as np
import pytest

from conftest import REPO

sys.path.insert(0, os.path.join(REPO, "tests", "golden"))
import make_golden  # noqa: E402

GOLDEN = os.path.join(REPO, "tests", "golden", "golden.npz")


@pytest.fixture(scope="module")
def committed():
    return dict(np.load(GOLDEN, allow_pickle=False))


def test_oracle_reproduces_golden(committed):
    fresh = make_golden.build()
    assert sorted(fresh) == sorted(committed)
    for k, v in committed.items():
        f = fresh[k]
        assert f.dtype == v.dtype and f.shape == v.shape, k
        assert np.array_equal(f.view(np.uint8), v.view(np.uint8)), k


def test_golden_inputs_follow_the_writer(committed, tmp_path):
    """The synthetic writer is deterministic: same config and seed, same bytes."""
    path = make_golden.model_file(str(tmp_path))
    assert hashlib.sha256(open(path, "rb").read()).digest() == committed["model.sha256"].tobytes()
