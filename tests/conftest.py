"""pytest configuration: the `gpu` marker and import paths.

Tests marked `gpu` need an MI355X (they call the HIP library through its C
ABI); everything else runs on the CPU.  The package directory has a hyphen in
its name, so its Python binding is imported from its path.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "serving-engine_amd")
for p in (ROOT, PKG, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD MI355X GPU and the built HIP library")
