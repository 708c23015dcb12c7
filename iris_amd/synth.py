"""Synthetic models, random-initialised from a seed.

Two generators:

* ``Xorshift32`` reproduces the reference's parity-bundle generators
  (model-bundles/parity-{gemma,mistral}/generate.py:35-199 / :87-271): the
  same integer xorshift32 sequence, tensor order and Q8_0 packing, so a
  regenerated ``model.detwgt`` is byte-identical to the checked-in one
  (pinned by its SHA-256).
* ``counter_hash`` is a counter-based splitmix64, vectorised in numpy: any
  row of any tensor can be generated on its own, so multi-GB configurations
  are generated on several threads and a checker can regenerate sampled rows.

Config builders cover the workloads this library is measured on: a tiny
gemma-dense model, Gemma-2B and Mistral-7B shapes, and small test shapes.
"""
from __future__ import annotations

import concurrent.futures as cf
import math
import os
import struct

import numpy as np

from . import detwgt
from .model import PREFIX, GemmaShape, MistralShape, Model
from .scalars import (ONE, attention_scale_q32, f32_to_acc_bits, f32_to_act_bits, f32_to_q16,
                      mistral_yarn_bounds, plain_rope_inverse_frequencies,
                      yarn_inverse_frequencies)

# ------------------------------------------------------------------ xorshift32


class Xorshift32:
    def __init__(self, seed: int):
        self.state = seed & 0xFFFFFFFF

    def next(self) -> int:
        s = self.state
        s ^= (s << 13) & 0xFFFFFFFF
        s ^= s >> 17
        s ^= (s << 5) & 0xFFFFFFFF
        self.state = s
        return s

    def values(self, count: int, amplitude: int, center: int = 0) -> list:
        out = []
        for _ in range(count):
            v = self.next() % (2 * amplitude) - amplitude
            out.append(center + (v if v else 1))
        return out

    def q8_blocks(self, count: int, scale_base: int) -> bytes:
        out = bytearray()
        for _ in range(count // 32):
            out += struct.pack("<H", scale_base + self.next() % 64)
            out += bytes((self.next() % 255 - 127) & 0xFF for _ in range(32))
        return bytes(out)


def parity_mistral_detwgt() -> bytes:
    """The reference's parity-mistral model.detwgt (seed 0x3A7E51C9)."""
    rng = Xorshift32(0x3A7E51C9)
    H, F, L, NH, KV, HD, V = 128, 2048, 4, 4, 2, 32, 512
    t = []
    t.append((PREFIX + "embed_tokens.weight", [V, H], 8, rng.q8_blocks(V * H, 0x1400)))
    t.append((PREFIX + "norm.weight", [H], 32, rng.values(H, 8192, ONE)))
    for layer in range(L):
        at = f"{PREFIX}layers.{layer}."
        for name, dims in [("self_attn.q_proj.weight", [NH * HD, H]),
                           ("self_attn.k_proj.weight", [KV * HD, H]),
                           ("self_attn.v_proj.weight", [KV * HD, H]),
                           ("self_attn.o_proj.weight", [H, NH * HD]),
                           ("mlp.gate_proj.weight", [F, H]),
                           ("mlp.up_proj.weight", [F, H]),
                           ("mlp.down_proj.weight", [H, F])]:
            t.append((at + name, dims, 8, rng.q8_blocks(math.prod(dims), 0x1000)))
        for name in ["input_layernorm.weight", "pre_feedforward_layernorm.weight"]:
            t.append((at + name, [H], 32, rng.values(H, 8192, ONE)))
    return detwgt.write(t)


def parity_mistral_shape() -> MistralShape:
    """Shape the importer derives from the bundle's config.json
    (crates/model/import/src/mistral.rs:202-289): YaRN factor 16, betas 32/1,
    original 16384 positions (also the position limit, since
    llama_4_scaling_beta is set), eps 1e-5, tied head."""
    hd = 32
    low, high = mistral_yarn_bounds(hd, 16384.0, 32.0, 1.0, 1_000_000.0)
    return MistralShape(
        hidden_size=128, num_hidden_layers=4, num_attention_heads=4, num_key_value_heads=2,
        head_dim=hd, intermediate_size=2048, vocab_size=512,
        norm_eps=f32_to_acc_bits(1e-5), attention_scale_q32=attention_scale_q32(hd),
        rope_inverse_frequencies=yarn_inverse_frequencies(1_000_000, hd // 2, 16, low, high),
        max_positions=16384, tied_head=True)


def parity_gemma_detwgt() -> bytes:
    """The reference's parity-gemma model.detwgt (seed 0x51A7E123)."""
    rng = Xorshift32(0x51A7E123)
    t = []
    t.append((PREFIX + "embed_tokens.weight", [512, 128], 8, rng.q8_blocks(512 * 128, 0x1000)))
    t.append((PREFIX + "embed_tokens_per_layer.weight", [512, 128], 8, rng.q8_blocks(512 * 128, 0x1400)))
    t.append((PREFIX + "per_layer_model_projection.weight", [128, 128], 32, rng.values(128 * 128, 4096)))
    t.append((PREFIX + "per_layer_projection_norm.weight", [32], 32, rng.values(32, 8192, ONE)))
    t.append((PREFIX + "norm.weight", [128], 32, rng.values(128, 8192, ONE)))
    t.append((PREFIX + "lm_head.weight", [512, 128], 8, rng.q8_blocks(512 * 128, 0x1400)))
    for layer in range(4):
        at = f"{PREFIX}layers.{layer}."
        for name, dims in [("self_attn.q_proj.weight", [128, 128]),
                           ("self_attn.k_proj.weight", [64, 128]),
                           ("self_attn.v_proj.weight", [64, 128]),
                           ("self_attn.o_proj.weight", [128, 128]),
                           ("mlp.gate_proj.weight", [2048, 128]),
                           ("mlp.up_proj.weight", [2048, 128]),
                           ("mlp.down_proj.weight", [128, 2048])]:
            t.append((at + name, dims, 8, rng.q8_blocks(math.prod(dims), 0x1000)))
        for name, dims in [("per_layer_input_gate.weight", [32, 128]),
                           ("per_layer_projection.weight", [128, 32])]:
            t.append((at + name, dims, 32, rng.values(math.prod(dims), 4096)))
        for name, width in [("input_layernorm.weight", 128), ("post_attention_layernorm.weight", 128),
                            ("pre_feedforward_layernorm.weight", 128),
                            ("post_feedforward_layernorm.weight", 128),
                            ("post_per_layer_input_norm.weight", 128),
                            ("self_attn.q_norm.weight", 32), ("self_attn.k_norm.weight", 32)]:
            t.append((at + name, [width], 32, rng.values(width, 8192, ONE)))
        t.append((at + "layer_scalar", [1], 32, [ONE]))
    return detwgt.write(t)


def gemma_shape(hidden, layers, heads, kv_heads, head_dim, vocab, ple_width, *, global_head_dim=None,
                sliding_window=0, layer_types=None, num_kv_shared_layers=0, eps=1e-6,
                rope_sliding=10_000, rope_full=1_000_000, partial_rotary=1.0, softcap=0.0,
                tied_head=True) -> GemmaShape:
    """A gemma-dense shape with the importer's scalar derivations
    (crates/model/import/src/gemma.rs:124-200, :725-756)."""
    f32 = np.float32
    return GemmaShape(
        hidden_size=hidden, num_hidden_layers=layers, num_attention_heads=heads,
        num_key_value_heads=kv_heads, head_dim=head_dim,
        global_head_dim=global_head_dim or head_dim, vocab_size=vocab,
        hidden_size_per_layer_input=ple_width, sliding_window=sliding_window,
        layer_types=list(layer_types or ["full_attention"] * layers),
        num_kv_shared_layers=num_kv_shared_layers, norm_eps=f32_to_acc_bits(eps),
        rope_base_sliding=int(rope_sliding) << 32, rope_base_full=int(rope_full) << 32,
        full_partial_rotary_factor_q16=f32_to_q16(partial_rotary),
        embedding_scale=f32_to_act_bits(float(np.sqrt(f32(hidden)))),
        ple_embedding_scale=f32_to_act_bits(float(np.sqrt(f32(ple_width)))),
        ple_projection_scalar=f32_to_act_bits(float(f32(hidden) ** f32(-0.5))),
        ple_input_scale=f32_to_act_bits(float(f32(2.0) ** f32(-0.5))),
        final_logit_softcap=f32_to_q16(softcap) if softcap else 0,
        tied_head=tied_head)


def parity_gemma_shape() -> GemmaShape:
    """Shape the importer derives from parity-gemma's config.json."""
    return gemma_shape(128, 4, 4, 2, 32, 512, 32, sliding_window=16,
                       layer_types=["sliding_attention", "full_attention"] * 2,
                       num_kv_shared_layers=2, eps=1e-6, rope_sliding=10_000, rope_full=1_000_000,
                       partial_rotary=0.5, softcap=1.0, tied_head=False)


# ------------------------------------------------------------------ counter hash

MASK64 = (1 << 64) - 1
GOLDEN = 0x9E3779B97F4A7C15
MIX1 = 0xBF58476D1CE4E5B9
MIX2 = 0x94D049BB133111EB


def splitmix64(x: np.ndarray) -> np.ndarray:
    """splitmix64's output function (Steele, Lea and Flood 2014) on uint64."""
    with np.errstate(over="ignore"):
        z = x.astype(np.uint64) + np.uint64(GOLDEN)
        z = (z ^ (z >> np.uint64(30))) * np.uint64(MIX1)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(MIX2)
        return z ^ (z >> np.uint64(31))


def tensor_seed(seed: int, tensor_id: int) -> int:
    return int(splitmix64(np.array([(seed * GOLDEN + tensor_id) & MASK64], dtype=np.uint64))[0])


def counter_hash(tseed: int, start: int, count: int) -> np.ndarray:
    """hash(tseed, i) for i in [start, start+count)."""
    with np.errstate(over="ignore"):
        idx = np.arange(start, start + count, dtype=np.uint64)
        return splitmix64(idx * np.uint64(GOLDEN) ^ np.uint64(tseed))


# (byte % 255) - 127 as an int8 bit pattern, for every byte value.
_Q_LUT = (((np.arange(256) % 255) - 127).astype(np.int8)).view(np.uint8)


def _q8_rows(tseed: int, r0: int, r1: int, nb: int, scale_base: int, per_row_scale: bool, out: np.ndarray):
    rows = r1 - r0
    h = counter_hash(tseed, r0 * nb * 4, rows * nb * 4)
    blk = out[r0:r1].reshape(rows, nb, 34)
    blk[:, :, 2:] = _Q_LUT[h.view(np.uint8).reshape(rows, nb, 32)]
    salt = tseed ^ 0x5CA1E5CA1E5CA1E5
    if per_row_scale:
        s = (counter_hash(salt, r0, rows) % np.uint64(64)).astype(np.int64) + scale_base
        s = np.broadcast_to(s[:, None], (rows, nb))
    else:
        s = ((counter_hash(salt, r0 * nb, rows * nb) % np.uint64(64)).astype(np.int64) + scale_base).reshape(rows, nb)
    blk[:, :, 0] = (s & 0xFF).astype(np.uint8)
    blk[:, :, 1] = (s >> 8).astype(np.uint8)


def q8_matrix(tseed: int, rows: int, cols: int, scale_base: int, per_row_scale: bool, threads: int = 0) -> np.ndarray:
    """Q8_0 bytes [rows, cols/32*34]: weights (byte % 255) - 127 from one hash
    per 8 weights (hash index (row*nb + block)*4 + j covers bytes 8j..8j+7 of
    the block); f16 scale bits ``scale_base + h % 64``, one per row
    (``per_row_scale``, every block of a row repeating it) or one per block.
    Rows are independent, so large matrices are generated on several threads."""
    nb = cols // 32
    out = np.empty((rows, nb * 34), dtype=np.uint8)
    threads = threads or min(16, os.cpu_count() or 1)
    chunk = max(1, -(-rows // (threads * 4)))
    if rows * nb < 65536 or threads == 1:
        _q8_rows(tseed, 0, rows, nb, scale_base, per_row_scale, out)
        return out
    with cf.ThreadPoolExecutor(threads) as ex:
        list(ex.map(lambda r0: _q8_rows(tseed, r0, min(rows, r0 + chunk), nb, scale_base, per_row_scale, out),
                    range(0, rows, chunk)))
    return out


def norm_vector(tseed: int, n: int) -> np.ndarray:
    """Q16.16 norm weights ONE + uniform[-8192, 8191]."""
    h = counter_hash(tseed, 0, n)
    return (ONE + (h % np.uint64(16384)).astype(np.int64) - 8192).astype(np.int32)


def i32_matrix(tseed: int, n: int, amplitude: int) -> np.ndarray:
    """Q16.16 values uniform in [-amplitude, amplitude)."""
    h = counter_hash(tseed, 0, n)
    return ((h % np.uint64(2 * amplitude)).astype(np.int64) - amplitude).astype(np.int32)


def f16_bits(x: float) -> int:
    return int(np.array([x], dtype=np.float16).view(np.uint16)[0])


def scale_base_for(cols: int) -> int:
    """f16 bits of about 1/(64*sqrt(cols)), minus half the jitter range, so a
    row times a unit-scale activation stays O(1)."""
    return f16_bits(1.0 / (64.0 * math.sqrt(cols))) - 32


class _Ids:
    def __init__(self):
        self.n = 0

    def __call__(self) -> int:
        self.n += 1
        return self.n


def mistral_model(hidden, layers, heads, kv_heads, head_dim, ffn, vocab, *, seed=0x1215, rope_base=1_000_000,
                  eps=1e-5, max_positions=32768, tied_head=False, per_row_scale=True,
                  eos_token_ids=()) -> Model:
    """A random-init mistral-dense model (plain RoPE = YaRN factor 1)."""
    shape = MistralShape(
        hidden_size=hidden, num_hidden_layers=layers, num_attention_heads=heads,
        num_key_value_heads=kv_heads, head_dim=head_dim, intermediate_size=ffn, vocab_size=vocab,
        norm_eps=f32_to_acc_bits(eps), attention_scale_q32=attention_scale_q32(head_dim),
        rope_inverse_frequencies=plain_rope_inverse_frequencies(rope_base, head_dim),
        max_positions=max_positions, tied_head=tied_head)
    ids = _Ids()
    t = {}
    emb_base = f16_bits(1.0 / 128.0) - 32
    t[PREFIX + "embed_tokens.weight"] = q8_matrix(tensor_seed(seed, ids()), vocab, hidden, emb_base, per_row_scale)
    t[PREFIX + "norm.weight"] = norm_vector(tensor_seed(seed, ids()), hidden)
    if not tied_head:
        t[PREFIX + "lm_head.weight"] = q8_matrix(tensor_seed(seed, ids()), vocab, hidden,
                                                 scale_base_for(hidden), per_row_scale)
    q, kv = heads * head_dim, kv_heads * head_dim
    for layer in range(layers):
        at = f"{PREFIX}layers.{layer}."
        for name, r, c in [("self_attn.q_proj.weight", q, hidden), ("self_attn.k_proj.weight", kv, hidden),
                           ("self_attn.v_proj.weight", kv, hidden), ("self_attn.o_proj.weight", hidden, q),
                           ("mlp.gate_proj.weight", ffn, hidden), ("mlp.up_proj.weight", ffn, hidden),
                           ("mlp.down_proj.weight", hidden, ffn)]:
            t[at + name] = q8_matrix(tensor_seed(seed, ids()), r, c, scale_base_for(c), per_row_scale)
        t[at + "input_layernorm.weight"] = norm_vector(tensor_seed(seed, ids()), hidden)
        t[at + "pre_feedforward_layernorm.weight"] = norm_vector(tensor_seed(seed, ids()), hidden)
    return Model("mistral-dense", shape, t, tuple(eos_token_ids))


def gemma_model(shape: GemmaShape, ffn: int, *, seed=0x6E33, per_row_scale=True, eos_token_ids=()) -> Model:
    """A random-init gemma-dense model over ``shape``."""
    s = shape
    ids = _Ids()
    t = {}
    H, P, L, V = s.hidden_size, s.hidden_size_per_layer_input, s.num_hidden_layers, s.vocab_size
    emb_base = f16_bits(1.0 / 512.0) - 32
    t[PREFIX + "embed_tokens.weight"] = q8_matrix(tensor_seed(seed, ids()), V, H, emb_base, per_row_scale)
    t[PREFIX + "embed_tokens_per_layer.weight"] = q8_matrix(tensor_seed(seed, ids()), V, L * P, emb_base,
                                                            per_row_scale)
    t[PREFIX + "per_layer_model_projection.weight"] = i32_matrix(tensor_seed(seed, ids()), L * P * H,
                                                                 4096).reshape(L * P, H)
    t[PREFIX + "per_layer_projection_norm.weight"] = norm_vector(tensor_seed(seed, ids()), P)
    t[PREFIX + "norm.weight"] = norm_vector(tensor_seed(seed, ids()), H)
    if not s.tied_head:
        t[PREFIX + "lm_head.weight"] = q8_matrix(tensor_seed(seed, ids()), V, H, scale_base_for(H), per_row_scale)
    for layer in range(L):
        at = f"{PREFIX}layers.{layer}."
        hd = s.head_dim if (layer < len(s.layer_types) and s.layer_types[layer] == "sliding_attention") \
            else s.global_head_dim
        q, kv = s.num_attention_heads * hd, s.num_key_value_heads * hd
        for name, r, c in [("self_attn.q_proj.weight", q, H), ("self_attn.k_proj.weight", kv, H),
                           ("self_attn.v_proj.weight", kv, H), ("self_attn.o_proj.weight", H, q),
                           ("mlp.gate_proj.weight", ffn, H), ("mlp.up_proj.weight", ffn, H),
                           ("mlp.down_proj.weight", H, ffn)]:
            t[at + name] = q8_matrix(tensor_seed(seed, ids()), r, c, scale_base_for(c), per_row_scale)
        t[at + "per_layer_input_gate.weight"] = i32_matrix(tensor_seed(seed, ids()), P * H, 4096).reshape(P, H)
        t[at + "per_layer_projection.weight"] = i32_matrix(tensor_seed(seed, ids()), H * P, 4096).reshape(H, P)
        for name, width in [("input_layernorm.weight", H), ("post_attention_layernorm.weight", H),
                            ("pre_feedforward_layernorm.weight", H), ("post_feedforward_layernorm.weight", H),
                            ("post_per_layer_input_norm.weight", H), ("self_attn.q_norm.weight", hd),
                            ("self_attn.k_norm.weight", hd)]:
            t[at + name] = norm_vector(tensor_seed(seed, ids()), width)
    return Model("gemma-dense", shape, t, tuple(eos_token_ids))


# ------------------------------------------------------------------ named workloads

def tiny_gemma(seed=0x71E7) -> Model:
    """2 layers, hidden 256, 4 heads of 64 with 1 KV head, GeGLU 1024, vocab
    4096, RoPE base 10000, PLE width 64, softcap 30."""
    shape = gemma_shape(256, 2, 4, 1, 64, 4096, 64, eps=1e-6, rope_sliding=10_000, rope_full=10_000,
                        softcap=30.0, tied_head=True)
    return gemma_model(shape, 1024, seed=seed)


def gemma4_e2b_scaled(seed=0x4E2B) -> Model:
    """The Gemma-4-E2B layout (runtime/model-artifacts/gemma-4-E2B-q8/
    manifest.json: 8 heads over 1 KV head, head size 256 on sliding layers
    and 512 on full ones, partial rotary 0.25 on the full layers, sliding
    window 512, KV-shared last layers, PLE width 256, softcap 30, RoPE bases
    10000 / 1e6) at a smaller hidden size and depth: hidden 256, 7 layers
    (four sliding, full, sliding, full; the last two KV-shared), GeGLU 512,
    vocab 2048, tied head."""
    shape = gemma_shape(256, 7, 8, 1, 256, 2048, 256, global_head_dim=512, sliding_window=512,
                        layer_types=["sliding_attention"] * 4 + ["full_attention", "sliding_attention",
                                                                 "full_attention"],
                        num_kv_shared_layers=2, eps=1e-6, rope_sliding=10_000, rope_full=1_000_000,
                        partial_rotary=0.25, softcap=30.0, tied_head=True)
    return gemma_model(shape, 512, seed=seed)


def gemma_2b(seed=0x2B2B) -> Model:
    """18 layers, hidden 2048, 8 heads of 256 with 1 KV head, GeGLU 16384,
    vocab 256000, RoPE base 10000, PLE width 256."""
    shape = gemma_shape(2048, 18, 8, 1, 256, 256000, 256, eps=1e-6, rope_sliding=10_000, rope_full=10_000,
                        softcap=30.0, tied_head=True)
    return gemma_model(shape, 16384, seed=seed)


MISTRAL_7B = dict(hidden=4096, layers=32, heads=32, kv_heads=8, head_dim=128, ffn=14336, vocab=32000)


def mistral_7b(seed=0x7B7B, layers=32, per_row_scale=True) -> Model:
    """32 layers, hidden 4096, 32 heads of 128 with 8 KV heads, SwiGLU 14336,
    vocab 32000, RoPE base 1e6, untied head; one f16 scale per row, or per
    block (``per_row_scale=False``: each block's own significand, the
    reference bundles' layout)."""
    kw = dict(MISTRAL_7B)
    kw["layers"] = layers
    return mistral_model(**kw, seed=seed, rope_base=1_000_000, eps=1e-5, max_positions=32768, tied_head=False,
                         per_row_scale=per_row_scale)


def token_ids(seed: int, count: int, vocab: int) -> np.ndarray:
    """Uniform prompt ids in [0, vocab)."""
    return (counter_hash(seed ^ 0x70C3, 0, count) % np.uint64(vocab)).astype(np.int64)
