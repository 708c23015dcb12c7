"""GPU parity past 4096 visible keys (the reference bounds a view only by
max_positions: crates/inference/kernels/src/mistral/layer.rs:121-127,
prefill_range.rs:755-845), through the C ABI.

Carried keys (iris_session_write_kv) fill every layer's cache up to a
position near 4096, past 2^15, or near the session bound of 65535; then a
multi-row range whose rows see the next 20 keys (the first case across the
one-tile bound of the row routines) and one-row ranges past it (the decode
kernels' tiled path) are compared with the oracle's layer over the same
keys, fed the device's rows of the layer below. Two attention shapes: four
query heads per KV head (the matrix-core prefill, whose exact value sums are
held in int32 up to 2^16 keys) and two (the one-row routine for every row).
"""
import numpy as np
import pytest

from iris_amd import native, synth
from iris_amd.direct import DeviceModel, Session
from oracle import cpu

pytestmark = pytest.mark.gpu

ROWS = 20
DECODE = 3


@pytest.fixture(scope="module", autouse=True)
def device():
    native.check(native.lib().q8gpu_init(), "q8gpu_init")


@pytest.mark.timeout(600)
@pytest.mark.parametrize("heads,kv_heads,CARRIED", [(8, 2, 4090), (4, 2, 4090), (8, 2, 40000), (8, 2, 65500),
                                                    (4, 2, 65500)])
def test_views_longer_than_one_tile_match_the_oracle(heads, kv_heads, CARRIED):
    m = synth.mistral_model(256, 2, heads, kv_heads, 64, 512, 1024, seed=71 + heads, max_positions=65536)
    n = CARRIED + ROWS + DECODE
    assert n <= 65535
    ids = synth.token_ids(72, n, m.vocab)
    kvw = kv_heads * 64
    rng = np.random.default_rng(73)
    carried = [(rng.integers(-(3 << 16), 3 << 16, (CARRIED, kvw)).astype(np.int32),
                rng.integers(-(3 << 16), 3 << 16, (CARRIED, kvw)).astype(np.int32)) for _ in range(m.num_layers)]
    print(f"heads {heads}/{kv_heads}: {CARRIED} carried keys, a {ROWS}-row range, {DECODE} one-row ranges",
          flush=True)
    dm = DeviceModel(m)
    s = Session(dm, n, ROWS)
    for layer, (k, v) in enumerate(carried):
        s.write_kv(layer, 0, k, v)
    r = cpu.OracleRun(m, n)
    for layer, (k, v) in enumerate(carried):
        r.k_cache[layer][:CARRIED] = k
        r.v_cache[layer][:CARRIED] = v
    seed = r.embed(list(ids))
    ranges = [(CARRIED, CARRIED + ROWS)] + [(p, p + 1) for p in range(CARRIED + ROWS, n)]
    for a, b in ranges:
        got, _ = s.layer_range(ids[a:b], a)
        x_prev = seed[a:b]
        for layer in range(m.num_layers):
            want = r.layer_pass(layer, x_prev, a, list(ids[a:b]), seed[a:b])
            assert np.array_equal(got[layer], want), f"range {a}..{b} layer {layer}"
            x_prev = got[layer]
        print(f"range {a}..{b}: {m.num_layers} layers equal", flush=True)
    for layer in range(m.num_layers):
        k, v = s.read_kv(layer, 0, n)
        assert np.array_equal(k, r.k_cache[layer][:n]) and np.array_equal(v, r.v_cache[layer][:n]), layer
    s.free()
    dm.free()


def test_session_position_bound():
    m = synth.mistral_model(256, 1, 8, 2, 64, 512, 1024, seed=74)
    dm = DeviceModel(m)
    s = Session(dm, 65535, 1)
    s.free()
    with pytest.raises(native.IrisError) as e:
        Session(dm, 65536, 1)
    assert e.value.code == -5  # IRIS_E_RANGE
    dm.free()
