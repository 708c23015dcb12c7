"""The direct-infer manifest contract and the mapped DETWGT load (no GPU).

- model_id_of against the ids the reference's own committed manifests hold
  (runtime/model-artifacts/*/manifest.json, in tests/golden/manifests.json);
- load_verified (crates/inference/artifacts/src/direct.rs:135-177) on a
  written bundle, and its refusals: a tampered weights / config / tokenizer
  file, another manifest version (the reference's own v2 manifest), an
  unknown family, a shape of the other family, an id that is not the hash of
  the commitments, a missing manifest;
- the mapped model equals the in-memory one, and tensors keep their keys.
"""
import json
import os

import numpy as np
import pytest

from iris_amd import artifacts, detwgt, model as model_mod, synth
from tests.conftest import golden


def test_model_id_of_matches_the_reference_manifests():
    fixtures = golden("manifests.json")["manifests"]
    checked = 0
    for name, m in fixtures.items():
        if m["model_id"] is None:
            continue
        assert artifacts.model_id_of(m["model_commitments"]) == m["model_id"], name
        checked += 1
    assert checked == 3
    # a dropped or reordered commitment changes the id
    m = fixtures["ministral-3b-q8"]
    c = m["model_commitments"]
    assert artifacts.model_id_of(c[1:]) != m["model_id"]
    assert artifacts.model_id_of([c[1], c[0]] + c[2:]) != m["model_id"]
    assert artifacts.model_id_of([]) == "e3b0c44298fc1c149afbf4c8996fb92427ae41e4649b934ca495991b7852b855"


def test_shape_family_of_the_reference_manifests():
    for name, m in golden("manifests.json")["manifests"].items():
        shape = {k: 0 for k in m["shape_fields"]}
        fam = artifacts.shape_family(shape)
        assert fam == (m["family"] or "gemma-dense"), name


def _bundle(tmp_path, family="mistral-dense"):
    if family == "mistral-dense":
        buf, shape = synth.parity_mistral_detwgt(), synth.parity_mistral_shape()
    else:
        buf, shape = synth.parity_gemma_detwgt(), synth.parity_gemma_shape()
    sd = {k: v for k, v in vars(shape).items()}
    if family == "gemma-dense":
        sd.pop("tied_head")
    commitments = [{"role": "decoder", "commitment": "ab" * 32}, {"role": "head", "commitment": "cd" * 32}]
    path = artifacts.write_bundle(str(tmp_path), buf, family, sd, eos_token_ids=[2], commitments=commitments,
                                  config={"text_config": {"tie_word_embeddings": bool(shape.tied_head)}})
    return path, buf, shape


def test_load_verified_accepts_a_written_bundle(tmp_path):
    path, _, _ = _bundle(tmp_path)
    m = artifacts.ModelManifest.load_verified(path)
    assert m.family == "mistral-dense" and m.version == 19 and m.eos_token_ids == [2]
    assert m.model_id == artifacts.model_id_of(m.model_commitments)


@pytest.mark.parametrize("victim,label", [("model.detwgt", "model weights"), ("config.json", "model config"),
                                          ("tokenizer.json", "model tokenizer")])
def test_a_tampered_file_is_refused(tmp_path, victim, label):
    path, _, _ = _bundle(tmp_path)
    f = os.path.join(str(tmp_path), victim)
    data = bytearray(open(f, "rb").read())
    data[len(data) // 2] ^= 1
    open(f, "wb").write(bytes(data))
    with pytest.raises(artifacts.ManifestError, match=f"{label} hash mismatch"):
        artifacts.ModelManifest.load_verified(path)


def _edit(path, **changes):
    d = json.load(open(path))
    d.update(changes)
    json.dump(d, open(path, "w"))


def test_refusals(tmp_path):
    path, _, _ = _bundle(tmp_path)
    good = json.load(open(path))
    _edit(path, version=2)  # the reference's own gemma-4-E2B-detwgt manifest is v2
    with pytest.raises(artifacts.ManifestError, match="unsupported model manifest v2, expected v19"):
        artifacts.ModelManifest.load_verified(path)
    json.dump(good, open(path, "w"))
    _edit(path, family="llama")
    with pytest.raises(artifacts.ManifestError, match="model family `llama` is not supported"):
        artifacts.ModelManifest.load_verified(path)
    json.dump(good, open(path, "w"))
    _edit(path, family="gemma-dense")
    with pytest.raises(artifacts.ManifestError, match="its shape is `mistral-dense`'s"):
        artifacts.ModelManifest.load_verified(path)
    json.dump(good, open(path, "w"))
    _edit(path, model_id="00" * 32)
    with pytest.raises(artifacts.ManifestError, match="model id does not match"):
        artifacts.ModelManifest.load_verified(path)
    with pytest.raises(artifacts.ManifestError, match="missing direct-infer manifest"):
        artifacts.load_model(os.path.join(str(tmp_path), "nothing.json"))


@pytest.mark.parametrize("family", ["mistral-dense", "gemma-dense"])
def test_mapped_model_equals_the_in_memory_one(tmp_path, family):
    path, buf, shape = _bundle(tmp_path, family)
    manifest, m, mapped = artifacts.load_model(path)
    want = model_mod.from_detwgt(buf, family, shape)
    assert m.family == family and sorted(m.tensors) == sorted(want.tensors)
    for name, t in want.tensors.items():
        assert np.array_equal(m.tensors[name], t), name
    assert vars(m.shape) == vars(shape)
    # keys name the bytes: (mapping, payload offset), distinct per tensor
    keys = {mapped.key(n) for n in mapped.tensors}
    assert len(keys) == len(mapped.tensors)
    name = next(iter(mapped.tensors))
    off = mapped.key(name)[1]
    assert open(mapped.path, "rb").read()[off:off + 16] == bytes(mapped.tensors[name].payload[:16])
    m.tensors = {}
    mapped.close()


def test_detwgt_reader_refusals():
    buf = synth.parity_mistral_detwgt()
    with pytest.raises(ValueError, match="truncated"):
        detwgt.read(buf[:-1])
    with pytest.raises(ValueError, match="trailing bytes"):
        detwgt.read(buf + b"\0")
    with pytest.raises(ValueError, match="not a detwgt"):
        detwgt.read(b"X" + buf[1:])
