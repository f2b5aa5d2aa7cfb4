"""The committed golden fixtures (tests/golden/*.npz) are reproduced by the
oracle: integer and byte outputs exactly, float outputs to 1e-9 relative
(fp64 reductions may reassociate across BLAS builds)."""
import os
import sys

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
import make_golden  # noqa: E402


@pytest.mark.parametrize("name", sorted(make_golden.FIXTURES))
def test_oracle_reproduces_fixture(name):
    stored = np.load(os.path.join(HERE, "golden", f"{name}.npz"))
    fresh = make_golden.generate(name)
    assert sorted(stored.files) == sorted(fresh)
    for key in stored.files:
        a, b = stored[key], np.asarray(fresh[key])
        assert a.dtype == b.dtype and a.shape == b.shape, key
        if a.dtype.kind == "f":
            fin = np.isfinite(a)
            assert np.array_equal(fin, np.isfinite(b)) and np.array_equal(a[~fin], b[~fin]), key
            np.testing.assert_allclose(b[fin], a[fin], rtol=1e-9, atol=1e-12, err_msg=key)
        else:
            assert np.array_equal(a, b), key
