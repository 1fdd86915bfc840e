"""Shared pytest configuration.

Markers:
  gpu  - needs an MI355X (gfx950) and the built HIP library; the driver runs
         these on the GPU box with ``-m gpu``.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP library")


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle as o
    o.build()
    return o


@pytest.fixture(scope="session")
def ref(orc):
    if not orc.ref_available():
        pytest.skip("oracle/_ref not built (reference sources absent when it was built)")
    return orc.ref()
