"""The round-end smoke check (__graft_entry__.smoke) runs as a GPU test too, so
a change to the chain's argument or workspace contract cannot leave it behind."""
from __future__ import annotations

import pytest

pytestmark = pytest.mark.gpu


def test_graft_entry_smoke(device):
    import __graft_entry__
    __graft_entry__.smoke()
