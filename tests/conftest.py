import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built liborca_hip.so")


@pytest.fixture(scope="session")
def ctx():
    from orcaml_amd.device import Context

    c = Context(0)
    yield c
    c.close()


@pytest.fixture(scope="session")
def hb(ctx):
    """HipBackend on the session's context."""
    from orcaml_amd.backend import HipBackend

    return HipBackend(ctx)
