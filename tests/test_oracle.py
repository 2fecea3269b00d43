"""The CPU oracle against its pins: closed forms, invariants, independent
library routines (numpy float16, scipy softmax, torch rms_norm / silu),
float64 brute force and the fixtures under tests/golden/."""
import pytest

import oracle_checks


@pytest.mark.parametrize("check", oracle_checks.ALL_CHECKS, ids=lambda c: c.__name__)
def test_oracle_pinned(oracle, check):
    fails = check(oracle)
    assert fails == [], "\n".join(fails)
