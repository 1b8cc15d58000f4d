# SPDX-License-Identifier: BSD-3-Clause
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and libxtc_hip.so")
    config.addinivalue_line("markers", "slow: long-running test")


def pytest_runtest_setup(item):
    # Print the test id before a GPU step so a crash names its case.
    if item.get_closest_marker("gpu") is not None:
        print(f"\n[gpu-test] {item.nodeid}", flush=True)
