"""The reference's direct-executor fixtures, built from their stated
construction (crates/inference/direct/tests/executor.rs):

* a gemma-dense model of no layers, 32 wide (one Q8_0 block per row), three
  token ids: embedding rows {0, e0, e1}, lm_head rows {0, 0, e0}, final norm
  ONE, norm_eps 0, no softcap, PLE width 1 (``write_tiny_model_detwgt``
  :639-661 and ``tiny_direct_manifest`` :663-707);
* the final-head tie: one row e0 against head rows {e0, 0, e0}
  (``final_head_logits_feed_shared_decode_select_tie_break`` :141-189).

e_i is the row with ONE at column i. Values are packed as exact Q8_0
blocks, each block taking the largest power-of-two scale that holds all its
values exactly (``q8_exact`` :792-810).
"""
from __future__ import annotations

import struct

from iris_amd import artifacts, detwgt
from iris_amd.model import PREFIX
from iris_amd.scalars import ONE

W = 32  # one Q8_0 block per row


def one_hot_rows(hot) -> list:
    """Rows W wide: an int column holds ONE, None is an all-zero row."""
    out = []
    for col in hot:
        out += [ONE if i == col else 0 for i in range(W)]
    return out


def q8_exact(values) -> bytes:
    """Whole 32-value blocks; each takes scale 2^-k (f16 bits (15-k) << 10)
    for the first k in 0..14 at which every value is a multiple of ONE >> k
    and the quotients fit in [-127, 127]."""
    out = bytearray()
    assert len(values) % 32 == 0, "Q8_0 rows are whole blocks"
    for b in range(0, len(values), 32):
        block = values[b:b + 32]
        for k in range(15):
            step = ONE >> k
            if all(v % step == 0 and abs(v // step) <= 127 for v in block):
                break
        else:
            raise ValueError("values are not exactly representable as Q8_0")
        out += struct.pack("<H", (15 - k) << 10)
        out += bytes((v // step) & 0xFF for v in block)
    return bytes(out)


def zero_layer_shape(vocab: int = 3) -> dict:
    """tiny_direct_manifest's gemma-dense shape (executor.rs:680-701)."""
    return {"hidden_size": W, "num_hidden_layers": 0, "num_attention_heads": 1, "num_key_value_heads": 1,
            "head_dim": 2, "global_head_dim": 2, "vocab_size": vocab, "hidden_size_per_layer_input": 1,
            "sliding_window": 0, "layer_types": [], "num_kv_shared_layers": 0, "norm_eps": 0,
            "rope_base_sliding": 10_000 << 32, "rope_base_full": 1_000_000 << 32,
            "full_partial_rotary_factor_q16": ONE, "embedding_scale": ONE, "ple_embedding_scale": ONE,
            "ple_projection_scalar": ONE, "ple_input_scale": ONE, "final_logit_softcap": 0}


def detwgt_bytes(embed_hot, head_hot) -> bytes:
    return detwgt.write([
        (PREFIX + "embed_tokens.weight", [len(embed_hot), W], 8, q8_exact(one_hot_rows(embed_hot))),
        (PREFIX + "lm_head.weight", [len(head_hot), W], 8, q8_exact(one_hot_rows(head_hot))),
        (PREFIX + "norm.weight", [W], 32, [ONE] * W),
    ])


TOKENIZER = {"model": {"type": "BPE", "vocab": {"<pad>": 0, "h": 1, "Hi": 2}, "merges": []}, "added_tokens": []}


def write_tiny_bundle(directory: str, eos_token_ids=()) -> str:
    """write_direct_fixture (executor.rs:620-637): the bundle and its
    manifest; returns the manifest's path. Prompt "h" is token 1."""
    return artifacts.write_bundle(directory, detwgt_bytes([None, 0, 1], [None, None, 0]), "gemma-dense",
                                  zero_layer_shape(), config={"text_config": {"tie_word_embeddings": False}},
                                  tokenizer=TOKENIZER, eos_token_ids=eos_token_ids)


def write_head_tie_bundle(directory: str) -> str:
    """The final-head tie as a loop: every token embeds to e0, head rows
    {e0, 0, e0}."""
    return artifacts.write_bundle(directory, detwgt_bytes([0, 0, 0], [0, None, 0]), "gemma-dense",
                                  zero_layer_shape(), config={"text_config": {"tie_word_embeddings": False}},
                                  tokenizer=TOKENIZER)
