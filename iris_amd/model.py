"""A model as the token loop sees it: a family, its shape scalars and its tensors.

Tensor names follow the reference's DETWGT naming
(crates/inference/direct/src/model.rs:489-588, import/src/*). Q8_0 matrices are
kept as their raw bytes (uint8 [rows, cols/32*34]); norm vectors and other
Q16.16 tensors as int32.

The shape types mirror inference_artifacts::{MistralShape, DirectInferShape}
(crates/inference/artifacts/src/direct.rs:241-290) and the per-layer derivations
of crates/inference/direct/src/model.rs:702-877.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from . import detwgt
from .scalars import ONE

PREFIX = "model.language_model."


@dataclass
class MistralShape:
    hidden_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    head_dim: int
    intermediate_size: int
    vocab_size: int
    norm_eps: int
    attention_scale_q32: int
    rope_inverse_frequencies: list
    max_positions: int
    tied_head: bool


@dataclass
class GemmaShape:
    hidden_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    head_dim: int
    global_head_dim: int
    vocab_size: int
    hidden_size_per_layer_input: int
    sliding_window: int
    layer_types: list
    num_kv_shared_layers: int
    norm_eps: int
    rope_base_sliding: int
    rope_base_full: int
    full_partial_rotary_factor_q16: int
    embedding_scale: int
    ple_embedding_scale: int
    ple_projection_scalar: int
    ple_input_scale: int
    final_logit_softcap: int
    tied_head: bool


@dataclass
class Model:
    family: str  # "mistral-dense" or "gemma-dense"
    shape: object
    tensors: dict = field(default_factory=dict)
    eos_token_ids: tuple = ()

    # ---- tensor access ----
    def q8(self, name: str) -> np.ndarray:
        return self.tensors[name]

    def values(self, name: str) -> np.ndarray:
        return self.tensors[name]

    def has(self, name: str) -> bool:
        return name in self.tensors

    @property
    def hidden(self) -> int:
        return self.shape.hidden_size

    @property
    def num_layers(self) -> int:
        return self.shape.num_hidden_layers

    @property
    def vocab(self) -> int:
        return self.shape.vocab_size

    def layer_name(self, layer: int, suffix: str) -> str:
        return f"{PREFIX}layers.{layer}.{suffix}"

    def embedding_name(self) -> str:
        return PREFIX + "embed_tokens.weight"

    def head_name(self) -> str:
        # model.rs:531-545: tied heads read the embedding table.
        return self.embedding_name() if self.shape.tied_head else PREFIX + "lm_head.weight"

    def final_norm(self) -> np.ndarray:
        return self.values(PREFIX + "norm.weight")

    def head_softcap(self) -> int:
        # model.rs:209-217: the mistral head is never capped.
        return self.shape.final_logit_softcap if self.family == "gemma-dense" else 0

    # ---- gemma per-layer derivations (crates/inference/direct/src/model.rs:817-877) ----
    def is_sliding(self, layer: int) -> bool:
        lt = self.shape.layer_types
        return layer < len(lt) and lt[layer] == "sliding_attention"

    def head_dim_at(self, layer: int) -> int:
        if self.family != "gemma-dense":
            return self.shape.head_dim
        return self.shape.head_dim if self.is_sliding(layer) else self.shape.global_head_dim

    def rope_at(self, layer: int):
        """(rope_base Q32.32, rotary_dim, rope_freq_base_dim) of a gemma layer."""
        hd = self.head_dim_at(layer)
        if self.is_sliding(layer):
            return self.shape.rope_base_sliding, hd, hd
        rotary = (hd * self.shape.full_partial_rotary_factor_q16) // ONE
        return self.shape.rope_base_full, int(rotary), hd

    def sliding_window_at(self, layer: int) -> int:
        return self.shape.sliding_window if self.is_sliding(layer) else 0

    def kv_donor_layer(self, layer: int) -> int:
        s = self.shape
        first_shared = max(s.num_hidden_layers - s.num_kv_shared_layers, 0)
        if s.num_kv_shared_layers == 0 or layer < first_shared:
            return -1
        if layer >= len(s.layer_types):
            return -1
        kind = s.layer_types[layer]
        for cand in range(first_shared - 1, -1, -1):
            if s.layer_types[cand] == kind:
                return cand
        return -1

    def layer_scalar(self, layer: int) -> int:
        name = self.layer_name(layer, "layer_scalar")
        if name in self.tensors and len(self.tensors[name]):
            return int(self.tensors[name][0])
        return 0

    def ffn_size(self, layer: int) -> int:
        return self.q8(self.layer_name(layer, "mlp.gate_proj.weight")).shape[0]


def from_detwgt(buf: bytes, family: str, shape, eos_token_ids=()) -> Model:
    """A model over a DETWGT artifact's tensors (Q8_0 kept raw)."""
    tensors = {}
    for name, t in detwgt.read(buf).items():
        tensors[name] = t.q8() if t.width == detwgt.Q8_0_WIDTH else t.values()
    return Model(family, shape, tensors, tuple(eos_token_ids))
