import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))

import __graft_entry__ as ge  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP device (MI355X)")


def _ensure_built():
    if not ge._built():
        ge.build()


_ensure_built()


@pytest.fixture(scope="session")
def pkg():
    return ge.load_package()


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle as o
    return o


@pytest.fixture(scope="session")
def ctx(pkg):
    c = pkg.MoeContext(0)
    yield c
    c.close()
