import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
TESTS = os.path.dirname(os.path.abspath(__file__))
for p in (ROOT, TESTS):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")
    config.addinivalue_line("markers", "slow: long-running CPU check")


def _banner(item):
    # Name the case before any GPU work starts, so a run that dies leaves a trace.
    if item.get_closest_marker("gpu"):
        print(f"\n[gpu-case] {item.nodeid}", flush=True)


def pytest_runtest_setup(item):
    _banner(item)
