"""The round-end smoke check (``__graft_entry__.smoke``) as a GPU test, so the suite
catches a smoke regression before the round-end run does."""

import pytest

pytestmark = pytest.mark.gpu


def test_graft_entry_smoke():
    import __graft_entry__

    __graft_entry__.smoke()
