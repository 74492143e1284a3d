import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def _print_case(item):
    # name the case before a GPU step runs, so a hard failure still says which one it was
    if item.get_closest_marker("gpu") is not None:
        print(f"\n[gpu case] {item.nodeid}", flush=True)


@pytest.hookimpl(tryfirst=True)
def pytest_runtest_setup(item):
    _print_case(item)
