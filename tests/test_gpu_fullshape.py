"""GPU parity at the full configurations, against the oracle.

- The teacher-forced chain pass at Mistral-7B shape over 2048 rows (the
  benchmark's model and ids): every layer is checked on its own, with the
  oracle fed the GPU's rows of the layer before. The oracle forms every row's
  keys and values (compared with the device's cache, all 2048 rows of every
  layer) and the layer output of sampled rows: 0, 31, 32, 127, 128, 1023,
  2047 and one random row in each 128-row tile. Each layer's SHA-256 is
  checked against its rows.
- The Mistral-7B-shape decode's 512-row prompt pass, layer by layer as
  above (every row's keys and values, sampled output rows, the first
  selection's logits), and the decode session's caches equal to that pass's.
- Mistral-7B-shape decode after the benchmark's 512-token prompt: 513
  greedy selections on the GPU (passes at positions 512..1023); the steps at
  positions 512, 767 and 1023 are each redone by the oracle from the device's
  own KV cache, and the step's own key/value rows of every layer and its
  logits must match.
- Gemma-2B-shape generation, a 128-token prompt and 256 greedy selections:
  every logit. The oracle runs the prompt and the 255 selected tokens as one
  batched pass (batched prefill equals the step-by-step decode for the
  oracle: tests/test_oracle_properties.py) and scores rows 127..382.

The oracle runs on the host's cores (OMP_NUM_THREADS of them when set); each
test prints its oracle time.
"""
import hashlib
import time

import numpy as np
import pytest

from iris_amd import native, synth
from iris_amd.direct import DeviceModel, Session
from oracle import cpu

pytestmark = pytest.mark.gpu

MISTRAL_7B_SEED = 0x7B7B  # the benchmark's model
PROMPT_SEED = 0x5EED      # the benchmark's prompt and teacher-forced ids


@pytest.fixture(scope="module", autouse=True)
def device():
    native.check(native.lib().q8gpu_init(), "q8gpu_init")


@pytest.fixture(scope="module")
def mistral_7b():
    m = synth.mistral_7b(seed=MISTRAL_7B_SEED)
    dm = DeviceModel(m)
    yield m, dm
    dm.free()


def sampled_rows(n, seed):
    rng = np.random.default_rng(seed)
    rows = {0, 31, 32, 127, 128, 1023, n - 1}
    rows |= {int(t * 128 + rng.integers(0, 128)) for t in range(n // 128)}
    return sorted(r for r in rows if r < n)


@pytest.mark.timeout(600)
def test_teacher_forced_2048_rows_at_mistral_7b_shape(mistral_7b):
    m, dm = mistral_7b
    n = 2048
    ids = synth.token_ids(PROMPT_SEED, n, m.vocab)
    s = Session(dm, n, n)
    rows, hashes = s.layer_pass(ids)
    sel = sampled_rows(n, 17)
    print(f"teacher-forced {n} rows done on the GPU; oracle over {len(sel)} sampled rows per layer", flush=True)
    r = cpu.OracleRun(m, n)
    x = r.embed(ids)
    t0 = time.time()
    for layer in range(m.num_layers):
        out = r.mistral_layer_rows(layer, x, 0, sel)
        assert np.array_equal(rows[layer][sel], out), f"layer {layer} rows"
        k, v = s.read_kv(layer, 0, n)
        assert np.array_equal(k, r.k_cache[layer][:n]), f"layer {layer} keys"
        assert np.array_equal(v, r.v_cache[layer][:n]), f"layer {layer} values"
        assert hashes[layer] == hashlib.sha256(rows[layer].astype("<i4").tobytes()).hexdigest()
        x = rows[layer]
    print(f"oracle: {time.time() - t0:.1f}s on {r.threads} threads", flush=True)
    s.free()


@pytest.fixture(scope="module")
def mistral_7b_decode(mistral_7b):
    """The benchmark's decode: a 512-token prompt, 513 greedy selections
    (passes at positions 512..1023), with the logits of every selection and
    every layer's cache afterwards."""
    m, dm = mistral_7b
    prompt = synth.token_ids(PROMPT_SEED, 512, m.vocab)
    s = Session(dm, 1024, 512)
    got = s.generate(prompt, 513, keep_logits=True)
    caches = [s.read_kv(layer, 0, 1024) for layer in range(m.num_layers)]
    s.free()
    return prompt, got, caches


@pytest.mark.timeout(600)
def test_mistral_7b_prompt_pass_against_the_oracle(mistral_7b, mistral_7b_decode):
    # The decode's 512-row prompt pass (the 128x64 matrix-core tiles with
    # their RoPE/KV-append, SwiGLU and residual epilogues, and the prefill
    # attention) layer by layer: the oracle is fed the device's rows of the
    # layer below and forms every row's keys and values and sampled output
    # rows; the last row's logits are the first selection's.
    m, dm = mistral_7b
    prompt, got, caches = mistral_7b_decode
    n = 512
    s = Session(dm, n, n)
    rows, hashes = s.layer_pass(prompt)
    for layer in range(m.num_layers):
        k, v = s.read_kv(layer, 0, n)
        assert np.array_equal(k, caches[layer][0][:n]), f"layer {layer}: decode session keys differ from the pass"
        assert np.array_equal(v, caches[layer][1][:n]), f"layer {layer}: decode session values differ from the pass"
    s.free()
    sel = sorted(set(sampled_rows(n, 29)) | {n - 1})
    print(f"prompt pass of {n} rows done on the GPU; oracle over {len(sel)} sampled rows per layer", flush=True)
    r = cpu.OracleRun(m, n)
    x = r.embed(prompt)
    t0 = time.time()
    for layer in range(m.num_layers):
        out = r.mistral_layer_rows(layer, x, 0, sel)
        assert np.array_equal(rows[layer][sel], out), f"layer {layer} rows"
        assert np.array_equal(caches[layer][0][:n], r.k_cache[layer][:n]), f"layer {layer} keys"
        assert np.array_equal(caches[layer][1][:n], r.v_cache[layer][:n]), f"layer {layer} values"
        assert hashes[layer] == hashlib.sha256(rows[layer].astype("<i4").tobytes()).hexdigest()
        x = rows[layer]
    logits = r.logits(rows[-1][n - 1])
    assert np.array_equal(got.logits[0], logits), "first selection's logits"
    assert got.token_ids[0] == int(np.argmax(logits))
    print(f"oracle: {time.time() - t0:.1f}s on {r.threads} threads", flush=True)


@pytest.mark.timeout(600)
def test_mistral_7b_decode_steps_from_the_device_cache(mistral_7b, mistral_7b_decode):
    m, dm = mistral_7b
    prompt, got, caches = mistral_7b_decode
    assert len(got.token_ids) == 513
    kvw = m.shape.num_key_value_heads * m.shape.head_dim
    r = cpu.OracleRun(m, 1024)
    t0 = time.time()
    for pos in (512, 767, 1023):
        step = pos - 512  # the pass at `pos` embeds selection `step` and gives selection step + 1
        for layer in range(m.num_layers):
            r.k_cache[layer][:pos] = caches[layer][0][:pos]
            r.v_cache[layer][:pos] = caches[layer][1][:pos]
        out, _ = r.pass_rows([got.token_ids[step]], pos)
        for layer in range(m.num_layers):
            assert np.array_equal(r.k_cache[layer][pos], caches[layer][0][pos]), f"pos {pos} layer {layer} key"
            assert np.array_equal(r.v_cache[layer][pos], caches[layer][1][pos]), f"pos {pos} layer {layer} value"
        logits = r.logits(out[-1])
        assert np.array_equal(got.logits[step + 1], logits), f"pos {pos} logits"
        assert got.token_ids[step + 1] == int(np.argmax(logits))
        print(f"decode step at position {pos}: keys, values and {logits.size} logits match ({kvw} kv)", flush=True)
    print(f"oracle: {time.time() - t0:.1f}s on {r.threads} threads", flush=True)


@pytest.mark.timeout(600)
def test_gemma_2b_prompt_128_and_256_selections():
    m = synth.gemma_2b()
    prompt = list(synth.token_ids(8, 128, m.vocab))
    dm = DeviceModel(m)
    s = Session(dm, 384, 128)
    got = s.generate(prompt, 256, keep_logits=True)
    assert len(got.token_ids) == 256
    print("gemma-2b shape: 256 selections on the GPU; oracle batched pass over 383 rows", flush=True)
    t0 = time.time()
    r = cpu.OracleRun(m, 384)
    rows, _ = r.pass_rows(prompt + got.token_ids[:255], 0)
    for i in range(256):
        logits = r.logits(rows[127 + i])
        assert np.array_equal(got.logits[i], logits), f"selection {i}"
        assert got.token_ids[i] == int(np.argmax(logits)), f"selection {i}"
    print(f"oracle: {time.time() - t0:.1f}s on {r.threads} threads", flush=True)
    s.free()
    dm.free()
