"""The oracle reproduces the committed golden fixtures (tests/golden/*.npz,
written by tests/golden/make_golden.py): integer outputs exactly, floating
outputs to 1e-6 relative L2 (the oracle accumulates some sums in parallel)."""
import os
import sys

import numpy as np
import pytest

from conftest import REPO, rel_l2

GOLDEN = os.path.join(REPO, "tests", "golden")
sys.path.insert(0, GOLDEN)


def _check(stored, fresh):
    assert sorted(stored.files) == sorted(fresh), "fixture keys changed"
    for k in stored.files:
        a, b = stored[k], np.asarray(fresh[k])
        assert a.shape == b.shape and a.dtype == b.dtype, k
        if np.issubdtype(a.dtype, np.integer):
            np.testing.assert_array_equal(a, b, err_msg=k)
        else:
            assert rel_l2(b, a) <= 1e-6, k


@pytest.mark.parametrize("name", ["raster_small.npz", "asm_small.npz", "geometry_small.npz"])
def test_oracle_reproduces_fixture(oracle_mod, name):
    import make_golden

    stored = np.load(os.path.join(GOLDEN, name))
    _check(stored, make_golden.FIXTURES[name]())
