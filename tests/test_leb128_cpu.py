"""Signed LEB128 oracle: the DWARF specification's worked examples (DWARF 4,
section 7.6, figure 23), round trips at the integer type limits."""

import numpy as np
import pytest

from oracle import leb128_oracle as leb

DWARF_SIGNED = [(2, b"\x02"), (-2, b"\x7e"), (127, b"\xff\x00"), (-127, b"\x81\x7f"), (128, b"\x80\x01"),
                (-128, b"\x80\x7f"), (129, b"\x81\x01"), (-129, b"\xff\x7e")]


@pytest.mark.parametrize("value,code", DWARF_SIGNED)
def test_dwarf_examples(value, code):
    assert leb.encode([value]) == code
    assert leb.decode(code, 1)[0] == value


def test_round_trip_at_type_limits():
    vals = np.array([0, 1, -1, 63, 64, -64, -65, 8191, 8192, -8192, -8193, 32767, -32768, 2**31 - 1, -2**31,
                     1048575, -1048576], np.int64)
    buf = leb.encode(vals)
    assert np.array_equal(leb.decode(buf, len(vals)), vals)
    g = np.random.default_rng(0)
    r = g.integers(-2**31, 2**31, 5000)
    assert np.array_equal(leb.decode(leb.encode(r), len(r)), r)


def test_code_lengths():
    # 7 value bits per byte, one of them the sign: 1 byte for [-64, 63], 2 for [-8192, 8191], ...
    for v, n in ((63, 1), (64, 2), (-64, 1), (-65, 2), (8191, 2), (8192, 3), (-8192, 2), (-8193, 3),
                 (32767, 3), (-32768, 3), (2**31 - 1, 5), (-2**31, 5)):
        assert len(leb.encode([v])) == n, v
