"""The committed golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py)
are reproduced bit-for-bit by the oracle, and their inputs are exact bf16 values."""
import importlib.util
from pathlib import Path

import numpy as np
import pytest

HERE = Path(__file__).resolve().parent / "golden"
spec = importlib.util.spec_from_file_location("make_golden", HERE / "make_golden.py")
make_golden = importlib.util.module_from_spec(spec)
spec.loader.exec_module(make_golden)


@pytest.mark.parametrize("name", sorted(make_golden.FIXTURES))
def test_fixture_is_reproduced(name):
    stored = np.load(HERE / (name + ".npz"))
    fresh = make_golden.build(name)
    assert set(stored.files) == set(fresh)
    for key in stored.files:
        np.testing.assert_array_equal(stored[key], np.asarray(fresh[key]), err_msg=key)


def test_bf16_rounding_is_round_to_nearest_even():
    one = 1.0
    x = np.array([one, one + 2 ** -8, one + 3 * 2 ** -9, one + 3 * 2 ** -8, -2.5], np.float32)
    r = make_golden.bf16(x)
    # bf16 spacing at 1 is 2^-7: a tie goes to the even neighbour, anything above it rounds up
    expect = np.array([one, one, one + 2 ** -7, one + 2 * 2 ** -7, -2.5], np.float32)
    np.testing.assert_array_equal(r, expect)
    assert (r.view(np.uint32) & 0xFFFF).max() == 0
