import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT / "google-classic_amd"))
sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs on the GPU box)")


@pytest.fixture(scope="session")
def oracle():
    from oracle.oracle import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def synth():
    from holo_mi355x import synth as s
    return s


@pytest.fixture(scope="session")
def holo():
    """The HIP library, initialised on device 0.  Only for tests marked gpu."""
    import holo_mi355x as h
    h.load()
    h.init()
    yield h
    h.check("end of session")
