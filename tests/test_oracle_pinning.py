"""The oracle passes every pinning check (reference test cases, float64 golden vectors,
invariants). CPU only."""

from __future__ import annotations

import pytest

from oracle import ref_cpu
from tests import pinning


@pytest.mark.parametrize("check", pinning.ALL_CHECKS, ids=lambda c: c.__name__)
def test_oracle_pinned(check):
    check(ref_cpu)
