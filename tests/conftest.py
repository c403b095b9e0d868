"""pytest configuration: the `gpu` marker and shared helpers.

Tests marked `gpu` need an MI355X and the built libwarppipe_mi355x.so; every
other test runs on the CPU (oracle vs golden vectors, host logic, library
loading and exports).
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a real MI355X GPU and the built HIP library")


@pytest.fixture(scope="session")
def golden_dir():
    return GOLDEN
