"""Pins the oracle functions no reference vector covers, through what the
mathematics fixes: closed forms, exact brute-force optima, symmetry, and
tolerance against the real functions the integer ones approximate. Each check
is chosen so a plausible transcription slip (a dropped Taylor term, a wrong
sign or rounding direction, a transposed operand) fails it."""
import ctypes as C
import math
from fractions import Fraction

import numpy as np
import pytest

from iris_amd import synth
from oracle import cpu

L = cpu.lib()
ONE = 1 << 16


def _rte(fr: Fraction) -> int:
    """Round a rational to the nearest integer, ties to even."""
    f = math.floor(fr)
    d = fr - f
    if d > Fraction(1, 2) or (d == Fraction(1, 2) and f % 2 == 1):
        return f + 1
    return f


def test_inv_sqrt_is_the_exact_optimum():
    # inv_sqrt_acc(x) = the u32 r minimising |r^2 x - 2^64| (ties to even),
    # capped at i32::MAX. Checked against its neighbours with exact integers.
    rng = np.random.default_rng(1)
    xs = [1, 2, 3, 4, 1 << 32, (1 << 32) + 1, 4294967296 * 7, (1 << 62) - 1, (1 << 63) - 1]
    xs += [int(v) for v in rng.integers(1, 1 << 62, 300)] + [int(v) for v in rng.integers(1, 1 << 20, 100)]
    for x in xs:
        r = L.dn_inv_sqrt_acc(x)
        if r == 2 ** 31 - 1:
            assert (2 ** 31 - 1) ** 2 * x <= 1 << 64 or x <= 4
            continue
        err = lambda c: abs(c * c * x - (1 << 64))
        assert err(r) <= err(r - 1) and err(r) <= err(r + 1), x
    assert L.dn_inv_sqrt_acc(0) == 2 ** 31 - 1


def test_rms_norm_closed_forms():
    # all-ONE rows with unit weights and eps 0 normalise to exactly ONE.
    for n in (4, 128, 4096):
        v = np.full(n, ONE, np.int32)
        assert (cpu.rms_norm(v, v, 0) == ONE).all()
    # Against the real RMSNorm within a few units.
    rng = np.random.default_rng(2)
    for n in (16, 256, 2048):
        v = rng.integers(-(8 << 16), 8 << 16, n).astype(np.int32)
        w = (ONE + rng.integers(-8192, 8192, n)).astype(np.int32)
        out = cpu.rms_norm(v, w, 4295)  # eps ~ 1e-6
        real = v / 65536.0 / np.sqrt(np.mean((v / 65536.0) ** 2) + 1e-6) * (w / 65536.0)
        assert np.abs(out / 65536.0 - real).max() <= 4 / 65536 * (1 + np.abs(real).max())


def test_softmax_exp_term_tracks_exp():
    worst = 0.0
    for d in np.linspace(-15.99, 0.0, 4001):
        delta = int(d * 2 ** 32)
        got = L.dn_softmax_exp_term(delta) / 2 ** 32
        worst = max(worst, abs(got - math.exp(delta / 2 ** 32)))
    # A 5th-order Taylor on r in [0, ln 2) errs by at most r^6/720 < 1.54e-4;
    # a dropped term would err by r^5/120 ~ 1.3e-3.
    assert worst < 1.6e-4, worst
    assert L.dn_softmax_exp_term(0) == 1 << 32
    assert L.dn_softmax_exp_term(-(16 << 32)) == 0


def test_softmax_closed_forms_and_tolerance():
    # n equal logits: each weight rte(rte(2^32/n)/2^16), residual to index 0.
    for n in (1, 2, 3, 7, 100):
        w = cpu.attention_softmax(np.full(n, 12345, np.int32))
        each = _rte(Fraction(_rte(Fraction(1 << 32, n)), 1 << 16))
        assert (w[1:] == each).all()
        assert w[0] == ONE - (n - 1) * each
    rng = np.random.default_rng(5)
    for n in (2, 17, 300):
        logits = rng.integers(-(12 << 16), 12 << 16, n).astype(np.int32)
        w = cpu.attention_softmax(logits)
        assert int(w.astype(np.int64).sum()) == ONE
        real = np.exp(logits / 65536.0 - (logits / 65536.0).max())
        real /= real.sum()
        assert np.abs(w / 65536.0 - real).max() < 3e-4
        # the residual lands on the first maximum
        ties = logits.copy()
        ties[-1] = ties.max()
        w2 = cpu.attention_softmax(ties)
        first = int(np.argmax(ties))
        assert w2[first] >= w2[-1]


def test_tanh_gelu_softcap_track_real_functions():
    xs = list(range(-(4 << 16), (4 << 16) + 1, 331))
    worst_t = worst_g = 0.0
    for x in xs:
        r = x / 65536.0
        t = L.dn_tanh_act(x)
        assert L.dn_tanh_act(-x) == -t  # odd, exactly
        worst_t = max(worst_t, abs(t / 65536.0 - math.tanh(r)))
        g = L.dn_gelu(x)
        real_g = 0.5 * r * (1 + math.tanh(math.sqrt(2 / math.pi) * (r + 0.044715 * r ** 3)))
        worst_g = max(worst_g, abs(g / 65536.0 - real_g))
    assert worst_t < 0.025, worst_t
    assert worst_g < 0.025, worst_g
    assert L.dn_tanh_act(3 << 16) == ONE and L.dn_tanh_act(-(3 << 16)) == -ONE
    cap = 30 << 16
    for x in range(-(60 << 16), 60 << 16, 7919):
        assert abs(L.dn_softcap_act(x, cap) / 65536.0 - 30 * math.tanh(x / 65536.0 / 30)) < 0.8


def test_sin_cos_acc_track_real_functions():
    worst = 0.0
    for a in np.linspace(-50.0, 50.0, 5001):
        c, s = cpu.sin_cos_acc(int(a * 2 ** 32))
        worst = max(worst, abs(c / 65536.0 - math.cos(a)), abs(s / 65536.0 - math.sin(a)))
    # Degree-6 cosine / degree-7 sine Taylor on [0, pi/2]: truncation at most
    # (pi/2)^8/8! = 9.19e-4; a dropped term would err by >= 2e-2.
    assert worst < 9.3e-4, worst


def test_nth_root_is_the_closest_power():
    for value, degree in [(10_000 << 32, 64), (1_000_000 << 32, 64), (10_000 << 32, 32), (2 << 32, 2),
                          (7 << 32, 3), (10_000 << 32, 128)]:
        r = L.dn_nth_root_acc(value, degree)
        assert abs(r / 2 ** 32 - (value / 2 ** 32) ** (1 / degree)) < 1e-6
        pw = lambda c: L.dn_pow_acc_u32(c, degree)
        e = lambda c: abs(pw(c) - value)
        assert e(r) <= e(r - 1) and e(r) <= e(r + 1)


def test_rope_frequency_ladder_tracks_powers():
    # The ladder's first pairs rotate at base^(-i/(d/2)).
    base, d = 10_000 << 32, 64
    step = L.dn_rope_frequency_step(base, d)
    assert abs(step / 2 ** 32 - 10_000 ** (-1 / 32)) < 1e-7


def test_mistral_trig_and_exp_track_real_functions():
    worst = 0.0
    for a in np.linspace(-40.0, 40.0, 4001):
        s, c = cpu.sin_cos_q30(int(a * 2 ** 32))
        worst = max(worst, abs(s / 2 ** 30 - math.sin(a)), abs(c / 2 ** 30 - math.cos(a)))
    assert worst < 1e-6, worst
    for a in np.linspace(0.0, 30.0, 601):
        e = L.dn_exp_neg_q32(int(a * 2 ** 32)) / 2 ** 32
        assert abs(e - math.exp(-a)) < 2e-9
    for x in range(-(20 << 16), 20 << 16, 4999):
        assert abs(L.dn_sigmoid_q32(x) / 2 ** 32 - 1 / (1 + math.exp(-x / 65536.0))) < 2e-9


def test_rotation_within_two_units_of_the_real_one():
    # crates/det-num/src/mistral.rs:241-258
    f = cpu.yarn_inverse_frequencies(1_000_000, 64, 16, 20, 37)
    for position in (1, 7, 513, 16383):
        v = np.array([(i - 64) * 9173 for i in range(128)], np.int32)
        out = cpu.rotate_consecutive_pairs(v, f, position)
        for p in range(64):
            ang = position * f[p] / 2 ** 32
            a, b = v[2 * p] / 65536.0, v[2 * p + 1] / 65536.0
            assert abs(out[2 * p] / 65536.0 - (a * math.cos(ang) - b * math.sin(ang))) <= 2 / 65536
            assert abs(out[2 * p + 1] / 65536.0 - (a * math.sin(ang) + b * math.cos(ang))) <= 2 / 65536


def _q8_row(rng, cols, max_exp):
    nb = cols // 32
    row = np.empty((nb, 34), np.uint8)
    v = rng.integers(0, 1 << 62, nb)
    bits = ((v & 1) << 15) | (((v >> 20) % (max_exp + 1)) << 10) | ((v >> 4) & 0x3FF)
    row[:, 0], row[:, 1] = bits & 0xFF, bits >> 8
    row[:, 2:] = rng.integers(0, 256, (nb, 32))
    return row.reshape(-1)


def _exact_dot_row(act, row) -> int:
    # sum of q * s * a / 2^40 over the whole row as one rational, rounded once.
    total = Fraction(0)
    blocks = row.reshape(-1, 34)
    for b, blk in enumerate(blocks):
        bits = int(blk[0]) | (int(blk[1]) << 8)
        e, m = (bits >> 10) & 31, bits & 1023
        s = Fraction(m, 1 << 24) if e == 0 else Fraction(1024 + m, 1 << 10) * Fraction(2) ** (e - 15)
        if bits & 0x8000:
            s = -s
        for j in range(32):
            total += int(np.int8(blk[2 + j])) * s * Fraction(int(act[b * 32 + j]), 1 << 16)
    return max(-2 ** 31, min(2 ** 31 - 1, _rte(total * (1 << 16))))


def test_dot_row_equals_the_exact_rational_product():
    rng = np.random.default_rng(9)
    for cols, max_exp, mag in [(32, 30, 31), (64, 18, 20), (96, 5, 12), (128, 30, 31)]:
        for _ in range(6):
            row = _q8_row(rng, cols, max_exp)
            act = (rng.integers(-(1 << 62), 1 << 62, cols) >> (63 - mag)).astype(np.int32)
            act[rng.integers(0, cols)] = 2 ** 31 - 1
            act[rng.integers(0, cols)] = -2 ** 31
            assert cpu.q8_dot_row(act, row) == _exact_dot_row(act, row)


def test_slab_product_equals_one_dot_row_per_value():
    # tensor.rs:655-705 shapes, with varied scales (tensor.rs:611-629 pattern).
    rng = np.random.default_rng(7)
    for rows, cols, tokens in [(200, 64, 11), (130, 96, 7), (64, 64, 3), (300, 32, 1), (1, 32, 5)]:
        w = np.stack([_q8_row(rng, cols, 10) for _ in range(rows)])
        x = rng.integers(-2 ** 31, 2 ** 31, (tokens, cols)).astype(np.int32)
        out = cpu.linear_q8(x, w)
        for t in range(tokens):
            for r in range(0, rows, 13):
                assert out[t, r] == cpu.q8_dot_row(x[t], w[r])


@pytest.mark.parametrize("family", ["mistral-dense", "gemma-dense"])
def test_batched_prefill_equals_chunked_decode(family):
    # direct/tests/executor.rs:190-350: chunks (0,1),(1,2),(2,3),(3,5) give
    # the same rows and keys as one pass over all five.
    if family == "mistral-dense":
        m = synth.mistral_model(128, 2, 4, 2, 32, 256, 512, seed=11)
    else:
        m = synth.gemma_model(synth.gemma_shape(128, 2, 4, 2, 32, 512, 32, sliding_window=3,
                                                layer_types=["sliding_attention", "full_attention"],
                                                partial_rotary=0.5, softcap=1.0), 256, seed=12)
    ids = [3, 17, 99, 5, 400]
    full = cpu.OracleRun(m, 16)
    rows_full, layers_full = full.pass_rows(ids, 0, keep_layers=True)
    chunked = cpu.OracleRun(m, 16)
    pieces = []
    for a, b in [(0, 1), (1, 2), (2, 3), (3, 5)]:
        r, layers = chunked.pass_rows(ids[a:b], a, keep_layers=True)
        pieces.append(layers)
    for layer in range(m.num_layers):
        got = np.concatenate([p[layer] for p in pieces])
        assert (got == layers_full[layer]).all()
        assert (chunked.k_cache[layer][:5] == full.k_cache[layer][:5]).all()
        assert (chunked.v_cache[layer][:5] == full.v_cache[layer][:5]).all()


def test_sampled_rows_equal_the_full_layer():
    # orc_mistral_layer_rows (every row's keys, the listed rows' outputs)
    # against the full forward, at position 0 and after carried keys.
    m = synth.mistral_model(128, 2, 4, 2, 32, 256, 512, seed=13)
    ids = list(synth.token_ids(14, 40, 512))
    full = cpu.OracleRun(m, 64)
    _, layers = full.pass_rows(ids, 0, keep_layers=True)
    _, layers_after = full.pass_rows(ids[:9], 40, keep_layers=True)
    sel = [0, 1, 17, 31, 39]
    part = cpu.OracleRun(m, 64)
    x = part.embed(ids)
    for layer in range(m.num_layers):
        out = part.mistral_layer_rows(layer, x, 0, sel)
        assert (out == layers[layer][sel]).all()
        assert (part.k_cache[layer][:40] == full.k_cache[layer][:40]).all()
        assert (part.v_cache[layer][:40] == full.v_cache[layer][:40]).all()
        x = layers[layer]
    x = part.embed(ids[:9])
    for layer in range(m.num_layers):
        out = part.mistral_layer_rows(layer, x, 40, [0, 4, 8])
        assert (out == layers_after[layer][[0, 4, 8]]).all()
        assert (part.k_cache[layer][:49] == full.k_cache[layer][:49]).all()
        x = layers_after[layer]


def test_gemma_embedding_scale_zero_gives_zero_rows():
    # model.rs:316-330: gemma-dense multiplies every embedded value by its
    # scale, zero included; mistral-dense leaves the row as dequantized.
    raw = synth.q8_matrix(synth.tensor_seed(15, 1), 4, 64, 0x3C00, False)
    out = np.empty(64, dtype=np.int32)
    assert cpu.lib().orc_embedding_row(raw[1], 64, 1, 0, out) == 0
    assert not out.any()
    assert cpu.lib().orc_embedding_row(raw[1], 64, 0, 0, out) == 0
    want = np.empty(64, dtype=np.int32)
    assert cpu.lib().dn_q8_dequantize_row(raw[1], 64, want) == 0
    assert (out == want).all() and want.any()
