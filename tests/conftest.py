import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))

GOLDEN = REPO / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def golden():
    import numpy as np

    cache = {}

    def load(name):
        if name not in cache:
            cache[name] = np.load(GOLDEN / f"{name}.npz")
        return cache[name]

    return load


@pytest.fixture(scope="session")
def tables():
    """The four cached L = 12 trellis tables of the reference (float64 x 4096)."""
    from lookatmyquant_amd.tables import load_table

    return {k: load_table(12, k) for k in (1, 2, 3, 4)}


@pytest.fixture(scope="session")
def config12():
    from lookatmyquant_amd import synthetic

    return synthetic.config12()
