"""GPU parity of the staged pass over ranges (the chain's layer stages with
carried keys), through the C ABI.

- Ranges reproduce the one-pass rows, hashes and keys bit for bit (batched
  prefill == chunked, docs/workflows/test-parity.md:137-138; the reference's
  chunked-vs-full check, crates/inference/direct/tests/executor.rs:190-350),
  for both families, with ranges that split 16-row query tiles and 64-key
  steps and a last one-row range.
- Keys carried into a fresh session (iris_session_write_kv) stand in for the
  earlier ranges' passes.
- One layer's stage (run_layer_stage, crates/inference/kernels/src/mistral/
  stage.rs:172-226) against the oracle's layer over the same carried keys,
  and the stage's output keys (carried ++ own, pruned to the window:
  prefill_range.rs:849-862).
- A range whose caches lack positions it needs is refused (the coverage
  check of raster-stages/layer-mistral/src/lib.rs:889-940).
"""
import hashlib

import numpy as np
import pytest

from iris_amd import model as model_mod, native, stage, synth
from iris_amd.direct import DeviceModel, Session
from oracle import cpu

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def device():
    native.check(native.lib().q8gpu_init(), "q8gpu_init")


def _model(family):
    if family == "mistral":
        # head size 64, four query heads per KV head: the matrix-core attention
        return synth.mistral_model(256, 3, 8, 2, 64, 512, 1024, seed=51)
    return model_mod.from_detwgt(synth.parity_gemma_detwgt(), "gemma-dense", synth.parity_gemma_shape())


CUTS = {"mistral": [0, 70, 131, 199, 200], "gemma": [0, 20, 37, 59, 60]}


def _full_pass(m, ids, n):
    dm = DeviceModel(m)
    s = Session(dm, n, n)
    rows, hashes = s.layer_pass(ids)
    keys = [s.read_kv(layer, 0, n) for layer in range(m.num_layers)]
    return dm, s, rows, hashes, keys


@pytest.mark.parametrize("family", ["mistral", "gemma"])
def test_ranges_reproduce_the_one_pass(family):
    m = _model(family)
    cuts = CUTS[family]
    n = cuts[-1]
    ids = synth.token_ids(61, n, m.vocab)
    print(f"{family}: one pass of {n} rows, then ranges {cuts}", flush=True)
    dm, s, rows, hashes, keys = _full_pass(m, ids, n)
    s2 = Session(dm, n, n)
    for a, b in zip(cuts, cuts[1:]):
        got, got_hashes = s2.layer_range(ids[a:b], a)
        for layer in range(m.num_layers):
            assert np.array_equal(got[layer], rows[layer][a:b]), f"range {a}..{b} layer {layer}"
            assert got_hashes[layer] == hashlib.sha256(rows[layer][a:b].astype("<i4").tobytes()).hexdigest()
    for layer in range(m.num_layers):
        k, v = s2.read_kv(layer, 0, n)
        assert np.array_equal(k, keys[layer][0]) and np.array_equal(v, keys[layer][1]), layer
    s2.free()
    s.free()
    dm.free()


@pytest.mark.parametrize("family", ["mistral", "gemma"])
def test_carried_keys_in_a_fresh_session(family):
    m = _model(family)
    n = CUTS[family][-1]
    a = CUTS[family][2]
    ids = synth.token_ids(62, n, m.vocab)
    dm, s, rows, hashes, keys = _full_pass(m, ids, n)
    s2 = Session(dm, n, n)
    with pytest.raises(native.IrisError) as e:
        s2.layer_range(ids[a:], a)
    assert e.value.code == -4  # IRIS_E_STATE: the keys before `a` are missing
    for layer in range(m.num_layers):
        s2.write_kv(layer, 0, keys[layer][0][:a], keys[layer][1][:a])
    got, _ = s2.layer_range(ids[a:], a)
    for layer in range(m.num_layers):
        assert np.array_equal(got[layer], rows[layer][a:]), layer
    # The chain API over KeyRow values: the same rows, and each layer's keys
    # carried ++ own (pruned to a sliding layer's window).
    s3 = Session(dm, n, n)
    prior = [stage.key_rows(keys[layer][0][:a], keys[layer][1][:a], 0) for layer in range(m.num_layers)]
    seqs = stage.run_chain_range(s3, ids[a:], a, prior)
    for layer, seq in enumerate(seqs):
        assert np.array_equal(seq.values(), rows[layer][a:]), layer
        w = m.sliding_window_at(layer) if m.family == "gemma-dense" else 0
        first = stage.window_start(a, w)
        assert [k.position for k in seq.kv] == list(range(first, n)), layer
        kk, vv = stage._key_arrays(seq.kv)
        assert np.array_equal(kk, keys[layer][0][first:]) and np.array_equal(vv, keys[layer][1][first:])
    for x in (s3, s2, s):
        x.free()
    dm.free()


@pytest.mark.parametrize("family", ["mistral", "gemma"])
def test_layer_stage_matches_the_oracle(family):
    m = _model(family)
    n = CUTS[family][-1]
    a = CUTS[family][1]
    ids = synth.token_ids(63, n, m.vocab)
    dm, s, rows, hashes, keys = _full_pass(m, ids, n)
    r = cpu.OracleRun(m, n)
    seed = r.embed(list(ids))
    s2 = Session(dm, n, n)
    x_prev = seed
    for layer in range(m.num_layers):
        # The oracle's layer over rows a..n with the one pass's keys before a.
        src = layer if family == "mistral" or m.kv_donor_layer(layer) < 0 else m.kv_donor_layer(layer)
        for cache_layer in {layer, src}:
            r.k_cache[cache_layer][:a] = keys[cache_layer][0][:a]
            r.v_cache[cache_layer][:a] = keys[cache_layer][1][:a]
        ple = None if family == "mistral" else r._ple_rows(layer, list(ids[a:]), seed[a:])
        want = r.layer_pass(layer, x_prev[a:], a, list(ids[a:]), seed[a:])
        assert np.array_equal(want, rows[layer][a:]), f"oracle layer {layer} vs the device one pass"
        # The device stage: carried keys as KeyRows, rows of the layer below.
        acts = stage.ActivationSequence(
            [stage.ActivationRow(int(t), x_prev[a + i].astype("<i4").tobytes()) for i, t in enumerate(ids[a:])],
            [], a)
        prior = stage.key_rows(keys[layer][0][:a], keys[layer][1][:a], 0)
        if src != layer:
            s2.write_kv(src, 0, keys[src][0][:a], keys[src][1][:a])
        out = stage.run_layer_stage(s2, layer, acts, prior, ple)
        assert not out.errors
        assert np.array_equal(out.values(), want), f"stage layer {layer}"
        w = m.sliding_window_at(layer) if m.family == "gemma-dense" else 0
        assert [k.position for k in out.kv] == list(range(stage.window_start(a, w), n))
        x_prev = rows[layer]
    # A stage whose carried keys leave a gap is refused: no rows, the cache
    # carried, the reason given.
    s3 = Session(dm, n, n)
    acts = stage.ActivationSequence(
        [stage.ActivationRow(int(t), seed[a + i].astype("<i4").tobytes()) for i, t in enumerate(ids[a:])], [], a)
    ple = None if family == "mistral" else r._ple_rows(0, list(ids[a:]), seed[a:])
    gap = stage.key_rows(keys[0][0][: a // 2], keys[0][1][: a // 2], 0)
    out = stage.run_layer_stage(s3, 0, acts, gap, ple)
    assert out.rows == [] and out.errors
    if family == "gemma":
        # A KV-shared layer's stage before its donor's stage over the same
        # range: the donor's cache lacks the range's own keys, so the stage
        # is refused rather than attending over stale keys.
        layer = next(l for l in range(m.num_layers) if m.kv_donor_layer(l) >= 0)
        src = m.kv_donor_layer(layer)
        s4 = Session(dm, n, n)
        s4.write_kv(src, 0, keys[src][0][:a], keys[src][1][:a])
        acts = stage.ActivationSequence(
            [stage.ActivationRow(int(t), rows[layer - 1][a + i].astype("<i4").tobytes())
             for i, t in enumerate(ids[a:])], [], a)
        ple = r._ple_rows(layer, list(ids[a:]), seed[a:])
        prior = stage.key_rows(keys[layer][0][:a], keys[layer][1][:a], 0)
        out = stage.run_layer_stage(s4, layer, acts, prior, ple)
        assert out.rows == [] and out.errors
        # after the donor's own stage over the range, the same stage runs
        donor_acts = stage.ActivationSequence(
            [stage.ActivationRow(int(t), (rows[src - 1] if src else seed)[a + i].astype("<i4").tobytes())
             for i, t in enumerate(ids[a:])], [], a)
        donor_prior = stage.key_rows(keys[src][0][:a], keys[src][1][:a], 0)
        stage.run_layer_stage(s4, src, donor_acts, donor_prior, r._ple_rows(src, list(ids[a:]), seed[a:]))
        out = stage.run_layer_stage(s4, layer, acts, prior, ple)
        assert not out.errors and np.array_equal(out.values(), rows[layer][a:])
        s4.free()
    for x in (s3, s2, s):
        x.free()
    dm.free()


def test_one_row_ranges_are_decode_passes():
    # A range of one row takes the one-row kernels (the decode path): the
    # last rows of a text as one-row ranges after a multi-row one.
    m = _model("mistral")
    n = 40
    ids = synth.token_ids(64, n, m.vocab)
    dm, s, rows, hashes, keys = _full_pass(m, ids, n)
    s2 = Session(dm, n, n)
    s2.layer_range(ids[:n - 3], 0, keep_rows=False)
    for p in range(n - 3, n):
        got, _ = s2.layer_range(ids[p:p + 1], p)
        for layer in range(m.num_layers):
            assert np.array_equal(got[layer], rows[layer][p:p + 1]), (p, layer)
    s2.free()
    s.free()
    dm.free()
