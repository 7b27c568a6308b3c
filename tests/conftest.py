import json
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP backend")


@pytest.fixture(scope="session")
def goldens():
    with open(os.path.join(GOLDEN, "reference_goldens.json")) as f:
        return json.load(f)


@pytest.fixture(scope="session")
def ora():
    import oracle

    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def hip():
    from graph_horizon_amd import HipBackend

    b = HipBackend(0)
    yield b
    b.close()


@pytest.fixture
def rng():
    return np.random.default_rng(1234)
