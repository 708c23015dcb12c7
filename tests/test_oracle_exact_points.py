"""The oracle's transcendental routines at inputs where the reference's own
arithmetic fixes every bit of the result, so that a misplaced floor, a wrong
rounding mode, a dropped term, a swapped quadrant sign or a shifted cutoff
in the restatement fails here (the reference holds no vectors for these
functions; their tolerance checks are in test_oracle_properties.py).

Each case follows from the reference's definitions
(crates/det-num/src/ops.rs, crates/det-num/src/mistral.rs), not from the
oracle's code:

* exp_neg_q32 (mistral.rs:43-56): a = k ln2 + r. For r = 0 every Horner step
  gives ONE, so e^-a = 2^32 >> k; for r = 1 only the n = 1 step subtracts
  (1 * ONE >> 32) / 1 = 1, so e^-a = (2^32 - 1) >> k; k >= 32 gives 0.
* sigmoid_q32 / silu (mistral.rs:59-77): sigmoid(0) = 2^63 / 2^33 << 1 =
  2^31; where exp_neg_q32 is 0 (|x| << 16 >= 32 ln2) the divisor is 2^32, so
  silu(x) = x for x >= 1453635 and 0 for x <= -1453635.
* softmax_exp_term (ops.rs:508-556): at delta = -k LN_2_BITS the Taylor
  sum is exactly ONE, giving 2^32 >> k (k <= 23; below -16 the term is 0);
  at delta = -(k LN_2_BITS + 1) it is ONE - 1, and the ties-to-even shift
  gives 2^32 - 1 for k = 0 and 2^(32-k) for k >= 1 (k = 1 is a tie).
* sin_cos_q30 (mistral.rs:84-109): for a reduced quarter angle q < 2^17,
  t = q >> 2 and u = t*t >> 30 = 0, so (sin, cos) = (t, 2^30) with the
  quadrant's signs; the four quadrants are reached at 0 + q, PI - q,
  PI + q and TWO_PI - q (the reference's constants).
* sin_cos_acc (ops.rs:622-683): for x <= 2^21 the cubic and higher terms
  round to 0 and the cosine's x^2/2 term to a value that requantizes to
  ONE, so (cos, sin) = (ONE, requantize(x)) with the quadrant's signs,
  requantize rounding ties to even (x = 32768 -> 0, x = 98304 -> 2).
* tanh_act (ops.rs:357-377): |x| <= 181 makes x^2 requantize to 0, so
  tanh(x) = div_act(27x, 27 ONE) = x; |x| >= 3 ONE saturates to +-ONE.
"""
import ctypes as C

import pytest

from oracle import cpu

LN2 = 2_977_044_472
ONE_Q32 = 1 << 32
ONE_Q30 = 1 << 30
ONE = 1 << 16
PI_Q32 = 13_493_037_705
TWO_PI_Q32 = 26_986_075_409


@pytest.fixture(scope="module")
def L():
    return cpu.lib()


def test_exp_neg_q32_at_zero_and_unit_remainders(L):
    for k in range(32):
        assert L.dn_exp_neg_q32(k * LN2) == ONE_Q32 >> k, k
        assert L.dn_exp_neg_q32(k * LN2 + 1) == (ONE_Q32 - 1) >> k, k
    for k in (32, 33, 40):
        assert L.dn_exp_neg_q32(k * LN2) == 0
        assert L.dn_exp_neg_q32(k * LN2 + 12345) == 0


def test_sigmoid_and_silu_where_the_exponential_vanishes(L):
    assert L.dn_sigmoid_q32(0) == 1 << 31
    edge = 1453635  # the least |x| with (|x| << 16) / LN2 >= 32
    assert (edge << 16) // LN2 >= 32 and ((edge - 1) << 16) // LN2 == 31
    for x in (edge, edge + 1, 5_000_000, 1 << 30, 2**31 - 1):
        assert L.dn_sigmoid_q32(x) == ONE_Q32
        assert L.dn_silu(x) == x
        assert L.dn_sigmoid_q32(-x) == 0
        assert L.dn_silu(-x) == 0
    # just inside the cutoff the exponential is still positive
    assert 0 < L.dn_sigmoid_q32(-(edge - 1))


def test_softmax_exp_term_at_zero_and_unit_remainders(L):
    for k in range(24):
        assert L.dn_softmax_exp_term(-k * LN2) == ONE_Q32 >> k, k
        want = ONE_Q32 - 1 if k == 0 else ONE_Q32 >> k
        assert L.dn_softmax_exp_term(-(k * LN2 + 1)) == want, k
    # at and below -16 (Acc) the term is 0
    assert L.dn_softmax_exp_term(-(16 << 32)) == 0
    assert L.dn_softmax_exp_term(-(16 << 32) - 1) == 0


def _sc_q30(L, angle):
    s, c = C.c_int64(), C.c_int64()
    L.dn_sin_cos_q30(angle, C.byref(s), C.byref(c))
    return s.value, c.value


@pytest.mark.parametrize("q", [0, 1, 3, 4, 5, 1000, 4097, 65535, (1 << 17) - 1])
def test_sin_cos_q30_small_quarter_angles_in_every_quadrant(L, q):
    t = q >> 2
    assert _sc_q30(L, q) == (t, ONE_Q30)
    assert _sc_q30(L, PI_Q32 - q) == (t, -ONE_Q30)
    assert _sc_q30(L, PI_Q32 + q) == (-t, -ONE_Q30)
    if q:
        assert _sc_q30(L, TWO_PI_Q32 - q) == (-t, ONE_Q30)
    # whole turns reduce to the same angle (rem_euclid), negative ones too
    assert _sc_q30(L, q + 3 * TWO_PI_Q32) == (t, ONE_Q30)
    assert _sc_q30(L, q - 2 * TWO_PI_Q32) == (t, ONE_Q30)


def _sc_acc(L, angle):
    c, s = C.c_int32(), C.c_int32()
    L.dn_sin_cos_acc(angle, C.byref(c), C.byref(s))
    return c.value, s.value


def _rte16(x):
    q, r = divmod(x, 1 << 16)
    return q + (1 if r > 1 << 15 or (r == 1 << 15 and q % 2) else 0)


@pytest.mark.parametrize("x", [0, 1, 32767, 32768, 32769, 98304, 163840, 1 << 20, 1 << 21])
def test_sin_cos_acc_small_angles_in_every_quadrant(L, x):
    s = _rte16(x)
    assert _sc_acc(L, x) == (ONE, s)
    assert _sc_acc(L, PI_Q32 - x) == (-ONE, s)
    assert _sc_acc(L, PI_Q32 + x) == (-ONE, -s)
    if x:
        assert _sc_acc(L, TWO_PI_Q32 - x) == (ONE, -s)


def test_sin_cos_acc_ties_to_even():
    assert _rte16(32768) == 0 and _rte16(98304) == 2 and _rte16(163840) == 2


def test_tanh_act_linear_range_and_saturation(L):
    for x in range(-181, 182):
        assert L.dn_tanh_act(x) == x, x
    for x in (3 * ONE, 3 * ONE + 1, 10 * ONE, 2**31 - 1):
        assert L.dn_tanh_act(x) == ONE
        assert L.dn_tanh_act(-x) == -ONE
    # approaching saturation the rational form stays at or below ONE
    assert all(L.dn_tanh_act(3 * ONE - d) <= ONE for d in range(1, 4097))
