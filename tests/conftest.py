import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) to run")


@pytest.fixture(scope="session")
def oracle():
    from oracle import refcpu
    refcpu.build()
    return refcpu


@pytest.fixture(scope="session")
def gn():
    import goneuron_amd as gn
    gn.GetDefaultDevice()
    return gn


@pytest.fixture(scope="session")
def dev(gn):
    return gn.GetDefaultDevice()
