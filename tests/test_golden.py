"""The NumPy oracle reproduces the committed golden fixtures exactly (CPU).

The fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py) are
the inputs and expected outputs the GPU golden tests compare against; this test
keeps the oracle and the files in step."""

import numpy as np
import pytest

from tests.golden import make_golden as G


@pytest.mark.parametrize("name", list(G.CASES))
def test_oracle_matches_fixture(name):
    ref = G.load(name)
    data = G.CASES[name]()
    assert set(data) == set(ref)
    for k, val in data.items():
        np.testing.assert_array_equal(np.asarray(val), ref[k], err_msg=f"{name}:{k}")
