"""The E4M3 restatement the FP8 cache tests rely on, pinned by brute force:
every encoded value is the nearest E4M3 value (ties to an even mantissa),
saturated at +-448."""

import numpy as np

from fp8_np import e4m3, e4m3_value, stored_position

GRID = e4m3_value(np.arange(0x7F))  # the 127 finite non-negative codes, increasing


def nearest_code(x: float) -> int:
    if x >= 448.0:
        return 0x7E
    d = np.abs(GRID - x)
    best = np.flatnonzero(d == d.min())
    return int(best[0] if len(best) == 1 else best[best % 2 == 0][0])


def test_grid_is_ocp_e4m3():
    assert GRID[0] == 0 and GRID[1] == 2.0 ** -9 and GRID[7] == 7 * 2.0 ** -9 and GRID[8] == 2.0 ** -6
    assert GRID[-1] == 448.0 and np.all(np.diff(GRID) > 0)
    assert np.isnan(e4m3_value(0x7F)) and np.isnan(e4m3_value(0xFF)) and e4m3_value(0x80) == 0.0


def test_e4m3_is_nearest_even_and_saturates():
    rng = np.random.default_rng(1)
    mids = (GRID[:-1] + GRID[1:]) / 2  # exact ties
    xs = np.concatenate([GRID, mids, np.nextafter(mids, 0), np.nextafter(mids, 1000), rng.uniform(0, 460, 5000),
                         np.exp(rng.uniform(-14, 6, 5000)), [464.0, 1e6, 448.0, 2.0 ** -10, 3 * 2.0 ** -10]])
    xs = xs.astype(np.float32).astype(np.float64)
    got = e4m3(xs.astype(np.float32))
    want = np.array([nearest_code(x) for x in xs], np.uint8)
    assert np.array_equal(got, want)
    assert np.array_equal(e4m3(-xs.astype(np.float32)), want | 0x80)


def test_stored_positions_are_a_permutation_of_groups():
    pos = stored_position(np.arange(16))
    assert sorted(pos) == list(range(16)) and list(pos[:8]) == [0, 1, 2, 3, 8, 9, 10, 11]
