import os
import sys

import pytest

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
from _pkg import load_oracle, load_pkg  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built libdpamd.so")


@pytest.fixture(scope="session")
def dp():
    return load_pkg()


@pytest.fixture(scope="session")
def orc():
    return load_oracle()
