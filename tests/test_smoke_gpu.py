"""The round-end smoke check (``__graft_entry__.smoke``) run as a GPU test, so that a change
to the decode path's outputs cannot leave it broken while the other tests pass."""

import importlib.util
from pathlib import Path

import pytest


@pytest.mark.gpu
def test_graft_entry_smoke():
    path = Path(__file__).resolve().parents[1] / "__graft_entry__.py"
    spec = importlib.util.spec_from_file_location("graft_entry_under_test", path)
    module = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(module)
    module.smoke()
