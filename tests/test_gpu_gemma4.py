"""GPU parity for the gemma-dense layout of the reference's gemma-4 models
(runtime/model-artifacts/gemma-4-E2B-q8/manifest.json), scaled down in
hidden size and depth: head size 256 on sliding layers and 512 on full
ones, partial rotary 0.25, a 512-key sliding window in use (a 600-token
text), KV-shared layers and PLE width 256. Every logit of greedy generation,
every layer's rows and hashes of the teacher-forced pass, and ranges of it
against the one pass, all against the oracle (the reference's attention
takes any head size: crates/inference/kernels/src/prefill_range.rs:755-845)."""
import hashlib

import numpy as np
import pytest

from iris_amd import native, synth
from iris_amd.direct import DeviceModel, Session
from oracle import cpu

pytestmark = pytest.mark.gpu

N = 600  # past the 512-key window


@pytest.fixture(scope="module", autouse=True)
def device():
    native.check(native.lib().q8gpu_init(), "q8gpu_init")


@pytest.fixture(scope="module")
def model():
    m = synth.gemma4_e2b_scaled()
    assert {m.head_dim_at(l) for l in range(m.num_layers)} == {256, 512}
    assert [m.kv_donor_layer(l) for l in range(m.num_layers)] == [-1, -1, -1, -1, -1, 3, 4]
    dm = DeviceModel(m)
    yield m, dm
    dm.free()


@pytest.fixture(scope="module")
def oracle_pass(model):
    m, _ = model
    ids = list(synth.token_ids(0x600, N, m.vocab))
    r = cpu.OracleRun(m, N + 8)
    rows, layers = r.pass_rows(ids, 0, keep_layers=True)
    return ids, r, rows, layers


def test_teacher_forced_pass_and_ranges(model, oracle_pass):
    m, dm = model
    ids, _, _, layers = oracle_pass
    print(f"gemma-4 layout: {N}-row pass", flush=True)
    s = Session(dm, N, N)
    rows, hashes = s.layer_pass(ids)
    for layer in range(m.num_layers):
        assert np.array_equal(rows[layer], layers[layer]), f"layer {layer} (head size {m.head_dim_at(layer)})"
        assert hashes[layer] == hashlib.sha256(layers[layer].astype("<i4").tobytes()).hexdigest()
    keys = [s.read_kv(layer, 0, N) for layer in range(m.num_layers)]
    # Ranges over the same text, the later ones past the window's reach.
    print("gemma-4 layout: ranges 0..250, 250..520, 520..599, 599..600", flush=True)
    s2 = Session(dm, N, N)
    cuts = [0, 250, 520, 599, N]
    for a, b in zip(cuts, cuts[1:]):
        got, _ = s2.layer_range(ids[a:b], a)
        for layer in range(m.num_layers):
            assert np.array_equal(got[layer], layers[layer][a:b]), f"range {a}..{b} layer {layer}"
    for layer in range(m.num_layers):
        k, v = s2.read_kv(layer, 0, N)
        assert np.array_equal(k, keys[layer][0]) and np.array_equal(v, keys[layer][1]), layer
    s2.free()
    s.free()


def test_long_pass_on_the_matrix_cores(model):
    # 1024 rows: 128 workgroups of 16 rows x 4 heads, from which the multi-row
    # attention runs on the matrix cores for head sizes 256 and 512 (the 600
    # rows above take the one-row routine). Every layer's rows against the
    # oracle, the sliding layers' 512-key window in use.
    m, dm = model
    n = 1024
    ids = list(synth.token_ids(0x1024, n, m.vocab))
    print(f"gemma-4 layout: {n}-row pass on the matrix cores", flush=True)
    _, layers = cpu.OracleRun(m, n).pass_rows(ids, 0, keep_layers=True)
    s = Session(dm, n, n)
    rows, _ = s.layer_pass(ids)
    for layer in range(m.num_layers):
        assert np.array_equal(rows[layer], layers[layer]), f"layer {layer} (head size {m.head_dim_at(layer)})"
    s.free()


@pytest.mark.parametrize("use_graph", [True, False])
def test_generation_every_logit(model, oracle_pass, use_graph):
    m, dm = model
    ids, r, rows, _ = oracle_pass
    tokens = 6
    print(f"gemma-4 layout: {N}-token prompt, {tokens} selections, graph={use_graph}", flush=True)
    s = Session(dm, N + 8, N)
    got = s.generate(ids, tokens, keep_logits=True, use_graph=use_graph)
    # The oracle's decode continues from its prompt pass (copies of its caches,
    # so that the other parametrisation starts from the same state).
    ks = [k.copy() for k in r.k_cache]
    vs = [v.copy() for v in r.v_cache]
    logits = r.logits(rows[-1])
    want_tokens, want_logits = [], []
    for t in range(tokens):
        want_logits.append(logits)
        tok = int(np.argmax(logits))
        want_tokens.append(tok)
        if t + 1 == tokens:
            break
        out, _ = r.pass_rows([tok], N + t)
        logits = r.logits(out[-1])
    for layer in range(m.num_layers):
        r.k_cache[layer][:] = ks[layer]
        r.v_cache[layer][:] = vs[layer]
    assert got.token_ids == want_tokens
    assert np.array_equal(got.logits, np.stack(want_logits))
    s.free()
