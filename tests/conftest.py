import json
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)

import __graft_entry__ as entry  # noqa: E402

# Measured errors of the GPU parity checks, one entry per check: the value,
# the bound the test asserts, and the headroom (bound / value).  Written at
# the end of the session to $Q38_MARGINS_PATH, by default
# gpurun_out/parity_margins.json (beside the run's other outputs).
_MARGINS = []


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device")


def pytest_sessionfinish(session, exitstatus):
    if not _MARGINS:
        return
    path = os.environ.get("Q38_MARGINS_PATH", os.path.join(ROOT, "gpurun_out", "parity_margins.json"))
    os.makedirs(os.path.dirname(path), exist_ok=True)
    with open(path, "w") as f:
        json.dump({"checks": _MARGINS}, f, indent=1)


@pytest.fixture
def margin(request):
    """margin(check, value, bound): record a measured error and assert
    value <= bound (NaN fails)."""

    def record(check: str, value: float, bound: float) -> None:
        value = float(value)
        _MARGINS.append({"test": request.node.nodeid, "check": check, "value": value, "bound": float(bound),
                         "headroom": (float(bound) / value) if value > 0 else None})
        print(f"[margin] {request.node.name} {check}: {value:.3e} (bound {bound:.0e})", flush=True)
        assert value <= bound, f"{check}: {value:.3e} > {bound:.3e}"

    return record


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
