"""Host logic of the staged pass (no GPU): the keys a range hands on
(crates/inference/kernels/src/prefill_range.rs:849-872) and the KeyRow
byte layout (little-endian int32 pages)."""
import numpy as np

from iris_amd import stage


def _keys(p0, n, width=3):
    k = np.arange(p0 * width, (p0 + n) * width, dtype=np.int32).reshape(n, width)
    return stage.key_rows(k, -k, p0)


def test_window_start():
    assert stage.window_start(0, 0) == 0
    assert stage.window_start(100, 0) == 0
    # a key is visible while query - key < window
    assert stage.window_start(15, 16) == 0
    assert stage.window_start(16, 16) == 1
    assert stage.window_start(100, 16) == 85


def test_output_kv_full_attention_carries_everything():
    prior, own = _keys(0, 20), _keys(20, 5)
    out = stage.output_kv(prior, own, 20, 0)
    assert [k.position for k in out] == list(range(25))


def test_output_kv_prunes_to_the_window_of_the_range_start():
    prior, own = _keys(0, 20), _keys(20, 5)
    out = stage.output_kv(prior, own, 20, 8)
    # keys before window_start(20, 8) = 13 are dropped; the range's own stay
    assert [k.position for k in out] == list(range(13, 25))
    # a range with no rows still carries the pruned cache
    assert [k.position for k in stage.output_kv(prior, [], 20, 8)] == list(range(13, 20))


def test_key_rows_are_little_endian_int32_pages():
    rows = _keys(7, 2, width=2)
    assert rows[0].position == 7 and rows[1].position == 8
    assert rows[0].k == np.array([14, 15], dtype="<i4").tobytes()
    assert rows[1].v == np.array([-16, -17], dtype="<i4").tobytes()
    k, v = stage._key_arrays(rows)
    assert k.tolist() == [[14, 15], [16, 17]] and v.tolist() == [[-14, -15], [-16, -17]]


def test_activation_sequence_values():
    vals = np.arange(12, dtype=np.int32).reshape(3, 4)
    seq = stage.ActivationSequence([stage.ActivationRow(i, vals[i].astype("<i4").tobytes()) for i in range(3)],
                                   [], 5)
    assert np.array_equal(seq.values(), vals)
