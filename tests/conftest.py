import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
HERE = os.path.dirname(os.path.abspath(__file__))
if HERE not in sys.path:
    sys.path.insert(0, HERE)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU; run on the GPU box")


@pytest.fixture(scope="session")
def engine():
    from seeker_amd import Engine

    e = Engine(0)
    yield e
    e.close()


def pytest_sessionfinish(session, exitstatus):
    """With SH_PARITY_LOG set, write every near-tie exemption the session took
    (tests/parity.py) as JSON: per kind the columns or cases compared and those
    that differed, and the per-test records."""
    path = os.environ.get("SH_PARITY_LOG")
    if not path:
        return
    import json

    import parity
    kinds = {}
    for r in parity.EXEMPTIONS:
        k = kinds.setdefault(r["kind"], {"compared": 0, "differing": 0, "checks": 0})
        k["compared"] += r["compared"]
        k["differing"] += r["differing"]
        k["checks"] += 1
    os.makedirs(os.path.dirname(os.path.abspath(path)), exist_ok=True)
    with open(path, "w") as f:
        json.dump({"exit_status": int(exitstatus), "kinds": kinds, "records": parity.EXEMPTIONS}, f, indent=1)
