"""Host-side helpers of the timing code (no GPU): the digit-plane count the
matrix-core products take for a set of activations, and the isolated
product's activation recipe."""
import numpy as np

from iris_amd import decode_timing


def _digits(v: int) -> int:
    # Signed byte digits d_l in [-128, 127] with v = sum d_l 256^l: the
    # fewest that represent v.
    for n in range(1, 6):
        lo, hi = -sum(128 * 256 ** l for l in range(n)), sum(127 * 256 ** l for l in range(n))
        if lo <= v <= hi:
            return n
    raise AssertionError(v)


def test_digit_planes_match_the_representation_bounds():
    edges = [0, 127, 128, -128, -129, 32639, 32640, -32896, -32897, 8355711, 8355712, -8421504, -8421505,
             0x7F7F7F7F, 0x7F7F7F80, -2 ** 31, 2 ** 31 - 1]
    rng = np.random.default_rng(1)
    vals = np.array(edges + list(rng.integers(-2 ** 31, 2 ** 31, 300)), dtype=np.int64)
    for v in vals:
        got = decode_timing.digit_planes_needed(np.array([[v]], dtype=np.int32))
        assert got.tolist() == [_digits(int(v))], int(v)


def test_digit_planes_per_token_group():
    x = np.zeros((300, 8), dtype=np.int32)
    x[5, 3] = 40000        # three digits in group 0
    x[130, 0] = -200       # two digits in group 1
    x[299, 7] = 2 ** 31 - 1  # five digits in the last, partial group
    assert decode_timing.digit_planes_needed(x).tolist() == [3, 2, 5]


def test_isolated_product_activations():
    x = decode_timing.c2_activations(64, 256, seed=2)
    assert x.shape == (64, 256) and x.dtype == np.int32
    assert np.abs(x).max() <= 127 * 511
    # each row is a multiple of its own scale in [256, 512)
    for row in x:
        g = int(np.gcd.reduce(np.abs(row[row != 0])))
        assert 256 <= g and g % 1 == 0 and any(g % s == 0 for s in range(256, 512))
