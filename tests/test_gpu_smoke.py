"""The round-end smoke check (``__graft_entry__.smoke``) runs in the GPU
suite too, so a change to the paths it exercises cannot leave it failing."""
import os
import sys

import pytest

pytestmark = pytest.mark.gpu

sys.path.insert(0, os.path.dirname(os.path.dirname(os.path.abspath(__file__))))


def test_smoke_entry_point():
    import __graft_entry__
    __graft_entry__.smoke()
