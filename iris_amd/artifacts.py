"""The direct-infer model manifest and its verified load.

Host-side mirror of inference_artifacts' direct-infer contract
(crates/inference/artifacts/src/direct.rs): ``manifest.json`` with its
version, family, model id and commitments, bundle paths and SHA-256s,
family shape and EOS ids; ``ModelManifest.load_verified``
(direct.rs:135-177) refuses a manifest of another version, a family this
build cannot run, a shape of another family, a model id that is not the
hash of its commitments (``model_id_of``, direct.rs:96-105) and any bundle
file whose SHA-256 (streamed, ``file_sha256`` direct.rs:209-225) differs
from the manifest's. ``load_model`` then maps the DETWGT file
(crates/model/detwgt/src/mmap.rs) and builds the model over the mapping,
as ``DirectInferenceModel::load`` does (crates/inference/direct/src/model.rs:
167-233).

Error messages follow the reference's wording.
"""
from __future__ import annotations

import hashlib
import json
import os
from dataclasses import dataclass, field

from . import detwgt
from .model import GemmaShape, MistralShape, Model

MODEL_MANIFEST_VERSION = 19
MODEL_MANIFEST_JSON = "manifest.json"
FAMILIES = ("gemma-dense", "mistral-dense")
MISSING_DIRECT_MANIFEST = "run iris model import ... to generate a model manifest"

_MISTRAL_FIELDS = ("hidden_size", "num_hidden_layers", "num_attention_heads", "num_key_value_heads", "head_dim",
                   "intermediate_size", "vocab_size", "norm_eps", "attention_scale_q32", "rope_inverse_frequencies",
                   "max_positions", "tied_head")
_GEMMA_FIELDS = ("hidden_size", "num_hidden_layers", "num_attention_heads", "num_key_value_heads", "head_dim",
                 "global_head_dim", "vocab_size", "hidden_size_per_layer_input", "sliding_window", "layer_types",
                 "num_kv_shared_layers", "norm_eps", "rope_base_sliding", "rope_base_full",
                 "full_partial_rotary_factor_q16", "embedding_scale", "ple_embedding_scale", "ple_projection_scalar",
                 "ple_input_scale", "final_logit_softcap")


class ManifestError(ValueError):
    pass


def model_id_of(commitments) -> str:
    """SHA-256 over each commitment's role, a zero byte, its commitment and
    a newline, in order (direct.rs:96-105)."""
    h = hashlib.sha256()
    for c in commitments:
        h.update(c["role"].encode())
        h.update(b"\0")
        h.update(c["commitment"].encode())
        h.update(b"\n")
    return h.hexdigest()


def file_sha256(path: str) -> str:
    """Streamed in 64 KiB reads, so large weight files use bounded memory."""
    h = hashlib.sha256()
    try:
        with open(path, "rb") as f:
            while True:
                chunk = f.read(64 * 1024)
                if not chunk:
                    break
                h.update(chunk)
    except OSError as e:
        raise ManifestError(f"failed to open {path}: {e}") from e
    return h.hexdigest()


def verify_file_sha256(path: str, expected: str, label: str) -> None:
    actual = file_sha256(path)
    if actual != expected:
        raise ManifestError(f"{label} hash mismatch for {path}: expected {expected}, got {actual}")


def shape_family(shape: dict) -> str:
    """The family whose shape this is (an untagged enum in the reference:
    mistral-dense's shape takes no unknown fields, direct.rs:261-290)."""
    if set(shape) == set(_MISTRAL_FIELDS):
        return "mistral-dense"
    if set(_GEMMA_FIELDS) <= set(shape):
        return "gemma-dense"
    raise ManifestError("model manifest shape is neither family's")


def resolve(manifest_dir: str, path: str) -> str:
    """model.rs:863-869: absolute paths as they are, others from the
    manifest's directory."""
    return path if os.path.isabs(path) else os.path.join(manifest_dir, path)


@dataclass
class ModelManifest:
    version: int
    family: str
    model_id: str
    model_commitments: list
    range_size: int
    bundle: dict
    shape: dict
    eos_token_ids: list
    provenance: dict | None = None
    path: str = field(default="", repr=False)

    @classmethod
    def from_json(cls, data: dict, path: str = "") -> "ModelManifest":
        try:
            return cls(version=int(data["version"]), family=data.get("family", FAMILIES[0]),
                       model_id=data["model_id"], model_commitments=list(data["model_commitments"]),
                       range_size=int(data["range_size"]), bundle=dict(data["bundle"]), shape=dict(data["shape"]),
                       eos_token_ids=[int(t) for t in data["eos_token_ids"]], provenance=data.get("provenance"),
                       path=path)
        except (KeyError, TypeError) as e:
            raise ManifestError(f"malformed model manifest {path}: {e}") from e

    def to_json(self) -> dict:
        out = {"version": self.version, "family": self.family, "model_id": self.model_id,
               "model_commitments": self.model_commitments, "range_size": self.range_size, "bundle": self.bundle,
               "shape": self.shape, "eos_token_ids": self.eos_token_ids}
        if self.provenance is not None:
            out["provenance"] = self.provenance
        return out

    def checked_family(self) -> str:
        if self.family not in FAMILIES:
            raise ManifestError(f"model family `{self.family}` is not supported by this build "
                                f"(supported: {', '.join(FAMILIES)})")
        return self.family

    @classmethod
    def load_verified(cls, path: str) -> "ModelManifest":
        """direct.rs:135-177."""
        try:
            with open(path) as f:
                data = json.load(f)
        except (OSError, ValueError) as e:
            raise ManifestError(f"failed to read {path}: {e}") from e
        m = cls.from_json(data, path)
        if m.version != MODEL_MANIFEST_VERSION:
            raise ManifestError(f"unsupported model manifest v{m.version}, expected v{MODEL_MANIFEST_VERSION}; "
                                "rerun a full `iris model import --model <bundle-dir>`")
        family = m.checked_family()
        if shape_family(m.shape) != family:
            raise ManifestError(f"model manifest says family `{family}` but its shape is "
                                f"`{shape_family(m.shape)}`'s")
        if m.model_id != model_id_of(m.model_commitments):
            raise ManifestError("model id does not match the manifest's model commitments")
        d = os.path.dirname(os.path.abspath(path))
        for key, label in (("config", "model config"), ("tokenizer", "model tokenizer"),
                           ("model_detwgt", "model weights")):
            verify_file_sha256(resolve(d, m.bundle[f"{key}_path"]), m.bundle[f"{key}_sha256"], label)
        return m

    def file(self, key: str) -> str:
        return resolve(os.path.dirname(os.path.abspath(self.path)), self.bundle[f"{key}_path"])


def family_shape(manifest: ModelManifest, tied_head: bool):
    s = manifest.shape
    if manifest.family == "mistral-dense":
        return MistralShape(**{k: s[k] for k in _MISTRAL_FIELDS})
    fields = {k: s[k] for k in _GEMMA_FIELDS}
    return GemmaShape(**fields, tied_head=tied_head)


def load_model(manifest_path: str):
    """(manifest, Model over the mapped DETWGT, the mapping): the weights are
    read from the mapping, not copied (DirectInferenceModel::load,
    crates/inference/direct/src/model.rs:167-233). The head is tied when
    config.json's text_config says tie_word_embeddings (model.rs:577-589)."""
    if not os.path.isfile(manifest_path):
        raise ManifestError(f"missing direct-infer manifest {manifest_path}; {MISSING_DIRECT_MANIFEST}")
    manifest = ModelManifest.load_verified(manifest_path)
    with open(manifest.file("config")) as f:
        config = json.load(f)
    text = config.get("text_config")
    if text is None:
        raise ManifestError("config.json has no text_config")
    tied = bool(text.get("tie_word_embeddings", False))
    mapped = detwgt.MappedDetwgt(manifest.file("model_detwgt"))
    tensors = {name: (t.q8() if t.width == detwgt.Q8_0_WIDTH else t.values()) for name, t in mapped.tensors.items()}
    model = Model(manifest.family, family_shape(manifest, tied), tensors, tuple(manifest.eos_token_ids))
    return manifest, model, mapped


def write_bundle(directory: str, model_bytes: bytes, family: str, shape: dict, *, config=None, tokenizer=None,
                 eos_token_ids=(), commitments=(), range_size=512) -> str:
    """Writes model.detwgt, config.json, tokenizer.json and
    runtime/model-artifacts/manifest.json (paths relative to it, as the
    reference's own fixtures do: direct/tests/executor.rs:372-470); returns
    the manifest's path."""
    os.makedirs(directory, exist_ok=True)
    files = {"model_detwgt": ("model.detwgt", model_bytes),
             "config": ("config.json", json.dumps(config or {"text_config": {"tie_word_embeddings": False}}).encode()),
             "tokenizer": ("tokenizer.json", json.dumps(tokenizer or {"model": {"type": "BPE", "vocab": {},
                                                                                "merges": []}}).encode())}
    bundle = {}
    for key, (name, data) in files.items():
        with open(os.path.join(directory, name), "wb") as f:
            f.write(data)
        bundle[f"{key}_path"] = os.path.join("..", "..", name)
        bundle[f"{key}_sha256"] = hashlib.sha256(data).hexdigest()
    art = os.path.join(directory, "runtime", "model-artifacts")
    os.makedirs(art, exist_ok=True)
    commitments = [dict(c) for c in commitments]
    m = ModelManifest(MODEL_MANIFEST_VERSION, family, model_id_of(commitments), commitments, range_size, bundle,
                      shape, list(eos_token_ids))
    path = os.path.join(art, MODEL_MANIFEST_JSON)
    with open(path, "w") as f:
        json.dump(m.to_json(), f, indent=2)
    return path
