"""Test setup: import paths for the package (hayate-exp_amd/) and the oracle,
and the `gpu` marker for tests that need an MI355X."""

import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for path in (ROOT, os.path.join(ROOT, "hayate-exp_amd")):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (MI355X, gfx950)")
