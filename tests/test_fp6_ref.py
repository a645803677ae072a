"""CPU: the reference e2m3 block encoder the fp6 GPU tests check against (tests/fp6_ref.py),
pinned by the format itself: every grid value encodes to its own code and decodes back, the
midpoints between neighbours round to the even code, rounding is monotone and never moves a
value by more than half a step, and the block exponent is the smallest that fits."""
import numpy as np

import fp6_ref as F


def test_grid_values_round_trip():
    for e in (-5, 0, 3):
        vals = F.E2M3_VALUES * 2.0 ** e
        for sign in (1.0, -1.0):
            code, val = F.encode((sign * vals).astype(np.float32), e)
            want = np.arange(32) | (32 if sign < 0 else 0)
            assert np.array_equal(code, want)
            assert np.array_equal(val, sign * vals)
            assert np.array_equal(F.decode(code, e), sign * vals)


def test_midpoints_round_to_even_code():
    v = F.E2M3_VALUES
    mids = (v[:-1] + v[1:]) / 2
    code, _ = F.encode(mids.astype(np.float32), 0)
    lo = np.arange(31)
    # of the two neighbours, the one with an even code (even mantissa) wins
    want = np.where(lo % 2 == 0, lo, lo + 1)
    assert np.array_equal(code, want)


def test_rounding_is_monotone_and_within_half_step():
    rng = np.random.default_rng(0)
    x = np.sort(rng.uniform(-7.5, 7.5, 200000).astype(np.float32))
    code, val = F.encode(x, 0)
    assert np.all(np.diff(val) >= 0)
    a = np.abs(x.astype(np.float64))
    step = np.where(a < 2, 0.125, np.where(a < 4, 0.25, 0.5))
    assert np.all(np.abs(val - x) <= step / 2 + 1e-12)


def test_block_exp_is_the_smallest_that_fits():
    rng = np.random.default_rng(1)
    bm = np.concatenate([rng.uniform(0, 1, 1000) * 10.0 ** rng.integers(-30, 30, 1000),
                         7.5 * 2.0 ** np.arange(-20, 20), 7.5 * 2.0 ** np.arange(-20, 20) * (1 + 2 ** -20)]).astype(np.float32)
    e = F.block_exp(bm)
    bm64 = bm.astype(np.float64)
    assert np.all(bm64 <= 7.5 * 2.0 ** e)
    assert np.all(bm64 > 7.5 * 2.0 ** (e - 1))
    assert F.block_exp(np.float32(0.0)) == 0
