import json
import pathlib
import sys

import numpy as np
import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
GOLDEN = ROOT / "tests" / "golden"
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device")


@pytest.fixture(scope="session")
def kats():
    return json.loads((GOLDEN / "kats.json").read_text())


@pytest.fixture(scope="session")
def session():
    """One rocm Session for all GPU tests; fails (never skips) without a device."""
    from affon_amd import Session
    s = Session("rocm")
    yield s
    s.dispose()


@pytest.fixture
def rng():
    return np.random.default_rng(20261105)
