"""Shared pytest setup: the ``gpu`` marker, the package import and small helpers."""
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

import __graft_entry__  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP extension")


@pytest.fixture(scope="session")
def pkg():
    return __graft_entry__.import_package()
