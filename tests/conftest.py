"""Shared pytest setup: import paths and the `gpu` marker."""

import os
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PACKAGE_ROOT = os.path.join(ROOT, "calibration-free-moe_amd")
for path in (ROOT, PACKAGE_ROOT):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line(
        "markers", "gpu: needs an MI355X (HIP device); run with -m gpu"
    )
