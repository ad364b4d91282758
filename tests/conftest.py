import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


def close(name, actual, expected, atol=3e-6, rtol=3e-5):
    """The reference's shared tolerance |a - e| < 3e-6 + 3e-5 |e| (src/library/src/tests.rs:5-20)."""
    import numpy as np

    a = np.asarray(actual, np.float64).reshape(-1)
    e = np.asarray(expected, np.float64).reshape(-1)
    assert a.shape == e.shape, f"{name}: shape {a.shape} != {e.shape}"
    assert np.all(np.isfinite(a)), f"{name}: non-finite values"
    err = np.abs(a - e)
    bad = err >= atol + rtol * np.abs(e)
    assert not bad.any(), (f"{name}: {int(bad.sum())} mismatches, first at {int(np.argmax(bad))}: "
                           f"{a[np.argmax(bad)]} != {e[np.argmax(bad)]}")
    return float(err.max()) if err.size else 0.0


@pytest.fixture(scope="session")
def oracle():
    from oracle import oracle as o

    o.build()
    return o
