"""GPU parity of the whole token loop against the oracle, through the C ABI:
every selected token and every logit the selection was made from, with and
without graph replay, for both families: small models, the reference's
parity bundle cases (EOS included), and the Mistral-7B and Gemma-2B shapes;
plus the teacher-forced per-layer pass (rows and per-layer SHA-256)."""
import hashlib
import os

import numpy as np
import pytest

from iris_amd import model as model_mod, native, synth
from iris_amd.direct import DeviceModel, Session
from oracle import cpu
from tests.conftest import golden

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def device():
    native.check(native.lib().q8gpu_init(), "q8gpu_init")


def _oracle_generate(m, prompt, tokens, max_pos):
    r = cpu.OracleRun(m, max_pos)
    return r.generate(list(prompt), tokens, keep_logits=True)


@pytest.mark.parametrize("use_graph", [True, False])
def test_small_mistral_generation_matches_oracle(use_graph):
    m = synth.mistral_model(128, 2, 4, 2, 32, 256, 512, seed=21, per_row_scale=False)
    prompt = synth.token_ids(3, 5, 512)
    print(f"small mistral, graph={use_graph}", flush=True)
    dm = DeviceModel(m)
    s = Session(dm, 64, 16)
    got = s.generate(prompt, 9, keep_logits=True, use_graph=use_graph)
    want_tokens, want_logits = _oracle_generate(m, prompt, 9, 64)
    assert got.token_ids == want_tokens
    assert np.array_equal(got.logits, np.stack(want_logits))


@pytest.mark.parametrize("use_graph", [True, False])
def test_timed_decode_generates_the_oracle_tokens(use_graph):
    # The benchmark's timed decode (graph replays or launch by launch):
    # the prompt's selection, then one token per timed step, as the oracle.
    m = synth.mistral_model(128, 2, 4, 2, 32, 256, 512, seed=23, per_row_scale=True)
    prompt = synth.token_ids(4, 7, 512)
    print(f"timed decode, graph={use_graph}", flush=True)
    dm = DeviceModel(m)
    s = Session(dm, 64, 16)
    ms, prefill, tokens = s.time_decode(prompt, 12, use_graph=use_graph)
    want_tokens, _ = _oracle_generate(m, prompt, 13, 64)
    # The oracle stops at an end-of-sequence id; the timed decode does not.
    assert tokens[:len(want_tokens)] == want_tokens
    assert len(want_tokens) == 13 or want_tokens[-1] in m.eos_token_ids
    assert ms > 0 and prefill > 0


@pytest.mark.parametrize("case", [0, 1, 2])
def test_parity_mistral_bundle_cases(case):
    g = golden("parity_bundles.json")["bundles"]["parity-mistral"]
    c = g["cases"][case]
    m = model_mod.from_detwgt(synth.parity_mistral_detwgt(), "mistral-dense", synth.parity_mistral_shape(),
                              eos_token_ids=g["eos_token_ids"])
    print(f"parity-mistral case {c['name']}", flush=True)
    dm = DeviceModel(m)
    s = Session(dm, 128, 64)
    got = s.generate(c["input_token_ids"], c["tokens"], keep_logits=True)
    want_tokens, want_logits = _oracle_generate(m, c["input_token_ids"], c["tokens"], 128)
    assert got.token_ids == want_tokens
    assert np.array_equal(got.logits, np.stack(want_logits))


def test_teacher_forced_layer_pass_matches_oracle():
    m = synth.mistral_model(256, 3, 8, 2, 32, 512, 1024, seed=22)
    ids = synth.token_ids(5, 40, 1024)
    dm = DeviceModel(m)
    s = Session(dm, 64, 64)
    rows, hashes = s.layer_pass(ids)
    r = cpu.OracleRun(m, 64)
    _, layers = r.pass_rows(list(ids), 0, keep_layers=True)
    for layer in range(m.num_layers):
        assert np.array_equal(rows[layer], layers[layer]), layer
        assert hashes[layer] == hashlib.sha256(layers[layer].astype("<i4").tobytes()).hexdigest()
    # The same pass without keeping the rows gives the same hashes.
    _, hashes2 = s.layer_pass(ids, keep_rows=False)
    assert hashes2 == hashes


def test_mistral_7b_shape_generation_matches_oracle():
    # The Mistral-7B shape (32 layers, hidden 4096, GQA 32/8, SwiGLU 14336,
    # vocab 32000): a short prompt and three selections, every logit
    # compared with the oracle.
    m = synth.mistral_7b(seed=0x7B7B)
    prompt = synth.token_ids(7, 4, 32000)
    print("mistral-7b shape: uploading", flush=True)
    dm = DeviceModel(m)
    s = Session(dm, 64, 8)
    got = s.generate(prompt, 3, keep_logits=True)
    print("mistral-7b shape: oracle", flush=True)
    want_tokens, want_logits = _oracle_generate(m, prompt, 3, 64)
    assert got.token_ids == want_tokens
    assert np.array_equal(got.logits, np.stack(want_logits))


# ---------------------------------------------------------------- gemma-dense

@pytest.mark.parametrize("case", [0, 1, 2])
def test_parity_gemma_bundle_cases(case):
    # Sliding layers (window 16) alternating with full ones, two KV-shared
    # layers, partial rotary on the full layers, softcap 1.0, untied head:
    # the cases run inside, across and past the window.
    g = golden("parity_bundles.json")["bundles"]["parity-gemma"]
    c = g["cases"][case]
    m = model_mod.from_detwgt(synth.parity_gemma_detwgt(), "gemma-dense", synth.parity_gemma_shape(),
                              eos_token_ids=g["eos_token_ids"])
    print(f"parity-gemma case {c['name']}", flush=True)
    dm = DeviceModel(m)
    s = Session(dm, 128, 64)
    got = s.generate(c["input_token_ids"], c["tokens"], keep_logits=True)
    want_tokens, want_logits = _oracle_generate(m, c["input_token_ids"], c["tokens"], 128)
    assert got.token_ids == want_tokens
    assert np.array_equal(got.logits, np.stack(want_logits))


@pytest.mark.parametrize("use_graph", [True, False])
def test_tiny_gemma_generation_matches_oracle(use_graph):
    # 2 layers, hidden 256, 4 heads of 64 over 1 KV head, GeGLU 1024, vocab
    # 4096, PLE 64, softcap 30: a 16-token prompt and 32 greedy selections.
    m = synth.tiny_gemma()
    prompt = synth.token_ids(11, 16, 4096)
    print(f"tiny gemma, graph={use_graph}", flush=True)
    dm = DeviceModel(m)
    s = Session(dm, 64, 16)
    got = s.generate(prompt, 32, keep_logits=True, use_graph=use_graph)
    want_tokens, want_logits = _oracle_generate(m, prompt, 32, 64)
    assert got.token_ids == want_tokens
    assert np.array_equal(got.logits, np.stack(want_logits))


def test_gemma_teacher_forced_layer_pass_matches_oracle():
    m = model_mod.from_detwgt(synth.parity_gemma_detwgt(), "gemma-dense", synth.parity_gemma_shape())
    ids = synth.token_ids(6, 40, m.vocab)
    dm = DeviceModel(m)
    s = Session(dm, 64, 64)
    rows, hashes = s.layer_pass(ids)
    r = cpu.OracleRun(m, 64)
    _, layers = r.pass_rows(list(ids), 0, keep_layers=True)
    for layer in range(m.num_layers):
        assert np.array_equal(rows[layer], layers[layer]), layer
        assert hashes[layer] == hashlib.sha256(layers[layer].astype("<i4").tobytes()).hexdigest()


def test_gemma_2b_shape_generation_matches_oracle():
    # The Gemma-2B configuration's shape (18 layers, hidden 2048, 8 heads of
    # 256 over 1 KV head, GeGLU 16384, vocab 256000, PLE 256, softcap 30):
    # a short prompt and three selections, every logit against the oracle.
    m = synth.gemma_2b()
    prompt = synth.token_ids(8, 4, m.vocab)
    print("gemma-2b shape: uploading", flush=True)
    dm = DeviceModel(m)
    s = Session(dm, 64, 8)
    got = s.generate(prompt, 3, keep_logits=True)
    print("gemma-2b shape: oracle", flush=True)
    want_tokens, want_logits = _oracle_generate(m, prompt, 3, 64)
    assert got.token_ids == want_tokens
    assert np.array_equal(got.logits, np.stack(want_logits))


# ---------------------------------------------------------------- selection and embedding edge cases

@pytest.mark.parametrize("per_row_scale", [True, False])
def test_tied_maxima_select_the_first_id(per_row_scale):
    # generation.rs:25-33, 63-64: the first maximum in id order wins. The head
    # holds one row w at ids 700 and 701 (one 16-row tile), 9000, 17000 and
    # 31000 (other tiles, other selection waves, the selection's second round
    # of tiles), its negation at 1300, 1301 and 20000, and zero rows
    # elsewhere: every step's maximum is shared by several ids.
    m = synth.mistral_model(256, 2, 4, 2, 64, 512, 32000, seed=23, per_row_scale=per_row_scale)
    head = m.tensors["model.language_model.lm_head.weight"]
    w = head[5].copy()
    blocks = w.copy().reshape(-1, 34)
    blocks[:, 2:] = (-(blocks[:, 2:].view(np.int8))).view(np.uint8)  # weights are in [-127, 127]
    new = np.zeros_like(head)
    for i in (700, 701, 9000, 17000, 31000):
        new[i] = w
    for i in (1300, 1301, 20000):
        new[i] = blocks.reshape(-1)
    m.tensors["model.language_model.lm_head.weight"] = new
    prompt = synth.token_ids(24, 6, m.vocab)
    dm = DeviceModel(m)
    s = Session(dm, 64, 8)
    got = s.generate(prompt, 12, keep_logits=True)
    want_tokens, want_logits = _oracle_generate(m, prompt, 12, 64)
    assert got.token_ids == want_tokens
    assert np.array_equal(got.logits, np.stack(want_logits))
    for logits in got.logits:
        assert np.count_nonzero(logits == logits.max()) >= 2
    assert set(got.token_ids) <= {0, 700, 1300}


def test_gemma_embedding_scale_zero():
    # model.rs:316-330 multiplies gemma-dense embeddings by their scale even
    # when it is zero: every embedded row is zero.
    import dataclasses
    m = synth.tiny_gemma()
    m.shape = dataclasses.replace(m.shape, embedding_scale=0)
    prompt = synth.token_ids(25, 5, m.vocab)
    dm = DeviceModel(m)
    s = Session(dm, 32, 8)
    got = s.generate(prompt, 4, keep_logits=True)
    want_tokens, want_logits = _oracle_generate(m, prompt, 4, 32)
    assert got.token_ids == want_tokens
    assert np.array_equal(got.logits, np.stack(want_logits))


@pytest.mark.parametrize("family,name", [("mistral-dense", "embed_tokens.weight"),
                                         ("gemma-dense", "embed_tokens_per_layer.weight")])
def test_non_finite_embedding_row_is_refused_when_embedded(family, name):
    # q8.rs:45-47: a Q8_0 scale with exponent 0x1f is not finite. The
    # reference dequantizes embedding rows when a token is embedded
    # (model.rs:316-330; the PLE prepare likewise), so a model with such a
    # row loads and runs; a prompt holding that token is refused.
    if family == "mistral-dense":
        m = synth.mistral_model(128, 1, 4, 2, 32, 256, 512, seed=26)
    else:
        m = synth.tiny_gemma()
    t = m.tensors["model.language_model." + name].copy()
    t[3, 0], t[3, 1] = 0x00, 0x7C  # token 3's first block: +inf
    m.tensors["model.language_model." + name] = t
    dm = DeviceModel(m)
    s = Session(dm, 32, 8)
    prompt = [5, 9, 2, 7]
    got = s.generate(prompt, 1, keep_logits=True)
    want_tokens, want_logits = _oracle_generate(m, prompt, 1, 32)
    assert got.token_ids == want_tokens
    assert np.array_equal(got.logits, np.stack(want_logits))
    with pytest.raises(native.IrisError) as e:
        s.generate([5, 3, 2], 1)
    assert e.value.code == -2


@pytest.mark.parametrize("family", ["mistral-dense", "gemma-dense"])
def test_model_from_a_verified_manifest(tmp_path, family):
    # A bundle written to disk, verified by its manifest, mapped and uploaded
    # tensor by tensor: generation equals the oracle over the same bytes.
    from iris_amd import artifacts
    if family == "mistral-dense":
        buf, shape, cases = synth.parity_mistral_detwgt(), synth.parity_mistral_shape(), "parity-mistral"
    else:
        buf, shape, cases = synth.parity_gemma_detwgt(), synth.parity_gemma_shape(), "parity-gemma"
    g = golden("parity_bundles.json")["bundles"][cases]
    sd = dict(vars(shape))
    if family == "gemma-dense":
        sd.pop("tied_head")
    path = artifacts.write_bundle(str(tmp_path), buf, family, sd, eos_token_ids=g["eos_token_ids"],
                                  config={"text_config": {"tie_word_embeddings": bool(shape.tied_head)}})
    dm = DeviceModel.from_manifest(path)
    assert dm.manifest.family == family
    c = g["cases"][2]
    s = Session(dm, 128, 64)
    got = s.generate(c["input_token_ids"], c["tokens"], keep_logits=True)
    m = model_mod.from_detwgt(buf, family, shape, eos_token_ids=g["eos_token_ids"])
    want_tokens, want_logits = _oracle_generate(m, c["input_token_ids"], c["tokens"], 128)
    assert got.token_ids == want_tokens
    assert np.array_equal(got.logits, np.stack(want_logits))
    s.free()
    dm.free()


def test_upload_cache_by_mapped_key(tmp_path):
    # Products over a mapped DETWGT through the drop-in ABI, uploads cached
    # by (mapping, offset): each matrix goes to the device once, and every
    # product equals the oracle's dot_row slab.
    from iris_amd import detwgt, tensor
    path = os.path.join(str(tmp_path), "model.detwgt")
    with open(path, "wb") as f:
        f.write(synth.parity_mistral_detwgt())
    mapped = detwgt.MappedDetwgt(path)
    cache = tensor.UploadCache()
    names = [n for n, t in mapped.tensors.items() if t.width == detwgt.Q8_0_WIDTH][:6]
    rng = np.random.default_rng(3)
    for rep in range(2):
        for n in names:
            raw = mapped.tensors[n].q8()
            rows, cols = raw.shape[0], raw.shape[1] // 34 * 32
            mat = cache.get(mapped.key(n), raw, rows, cols)
            x = rng.integers(-(1 << 20), 1 << 20, (3, cols)).astype(np.int32)
            assert np.array_equal(tensor.linear_slab_from_source(x, mat), cpu.linear_q8(x, raw)), n
    assert cache.uploads == len(names)
    cache.clear()
    mapped.close()


def test_per_block_teacher_forced_pass_matches_oracle():
    # Per-block scale matrices (the reference bundles' layout) in a multi-row
    # pass: every product runs folded on the matrix cores (q|k|v with the
    # RoPE/KV epilogue, SwiGLU pairs, residuals); every layer's rows and
    # hashes against the oracle.
    m = synth.mistral_model(512, 2, 8, 2, 64, 1024, 2048, seed=23, per_row_scale=False)
    ids = synth.token_ids(8, 300, 2048)
    dm = DeviceModel(m)
    s = Session(dm, 300, 300)
    rows, hashes = s.layer_pass(ids)
    r = cpu.OracleRun(m, 300)
    _, layers = r.pass_rows(list(ids), 0, keep_layers=True)
    for layer in range(m.num_layers):
        assert np.array_equal(rows[layer], layers[layer]), layer
        assert hashes[layer] == hashlib.sha256(layers[layer].astype("<i4").tobytes()).hexdigest()
    s.free()
    dm.free()
