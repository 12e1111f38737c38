"""The committed golden fixtures (tests/golden/*.npz) are reproduced bit for bit by the oracle from
their seeded inputs, and the inputs themselves still hash to the recorded digest."""
import os
import sys

import numpy as np
import pytest

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
sys.path.insert(0, GOLDEN)
import cases  # noqa: E402


@pytest.mark.parametrize("name", cases.CASES)
def test_oracle_reproduces_fixture(name):
    stored = np.load(os.path.join(GOLDEN, f"{name}.npz"))
    inputs, outputs = cases.build(name)
    assert str(stored["input_sha256"]) == cases.digest(inputs), "seeded inputs changed"
    for k, v in outputs.items():
        assert np.array_equal(stored[k], v, equal_nan=True), f"{name}.{k} differs from the fixture"
