import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import __graft_entry__ as entry  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device")


@pytest.fixture(scope="session")
def pkg():
    return entry.load_package()


@pytest.fixture(scope="session")
def ref():
    return entry.load_oracle()


@pytest.fixture(scope="session")
def synth(pkg):
    from q38amd import synth as s
    return s


@pytest.fixture(scope="session")
def ctx(pkg):
    c = pkg.Context(0)
    print(f"\n[gpu] {c.info()}", flush=True)
    yield c
    c.close()
