"""CPU oracle driver: ctypes bindings to liboracle.so and the reference's token
loop restated over them.

TEST INFRASTRUCTURE ONLY. Tests, ``__graft_entry__.smoke()`` and the
benchmark's ``cpu_baseline`` leg use this as the expected result / CPU baseline; the
shipped package never imports it.

The loop follows crates/inference/direct/src/executor.rs:143-185 (prefill all
prompt rows at position 0, then select / stop / embed / one-row pass per
token), run_layers_and_logits :293-360 (gemma: PLE prepare then the layer, per
layer, with KV donors) and run_mistral_layers_and_logits :364-401.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

_lib = None


def default_threads() -> int:
    """Host threads for the oracle: the CPU count, capped by OMP_NUM_THREADS
    when it is set (the share of the host a run is given)."""
    n = os.cpu_count() or 1
    env = os.environ.get("OMP_NUM_THREADS", "")
    return max(1, min(n, int(env))) if env.isdigit() and int(env) > 0 else n


def build() -> str:
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = C.CDLL(LIB_PATH)
        _declare(_lib)
    return _lib


i32p = np.ctypeslib.ndpointer(np.int32, flags="C_CONTIGUOUS")
i64p = np.ctypeslib.ndpointer(np.int64, flags="C_CONTIGUOUS")
u8p = np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS")
u32p = np.ctypeslib.ndpointer(np.uint32, flags="C_CONTIGUOUS")


class MistralLayerC(C.Structure):
    _fields_ = [("hidden", C.c_uint32), ("ffn", C.c_uint32), ("heads", C.c_uint32),
                ("kv_heads", C.c_uint32), ("head_dim", C.c_uint32), ("norm_eps", C.c_int64),
                ("attention_scale_q32", C.c_uint32), ("inv_freq", C.c_void_p),
                ("max_positions", C.c_uint32), ("norm_attention", C.c_void_p),
                ("norm_feed_forward", C.c_void_p)] + [
        (n, C.c_void_p) for n in ("w_q", "w_k", "w_v", "w_o", "w_gate", "w_up", "w_down")]


class GemmaLayerC(C.Structure):
    _fields_ = [("hidden", C.c_uint32), ("ffn", C.c_uint32), ("heads", C.c_uint32),
                ("kv_heads", C.c_uint32), ("head_dim", C.c_uint32), ("ple_width", C.c_uint32),
                ("sliding_window", C.c_uint32), ("layer_scalar", C.c_int32), ("norm_eps", C.c_int64),
                ("rope_base", C.c_int64), ("rotary_dim", C.c_uint32), ("rope_freq_base_dim", C.c_uint32)] + [
        (n, C.c_void_p) for n in ("norm_input", "norm_post_attn", "norm_pre_ffw", "norm_post_ffw",
                                  "q_norm", "k_norm", "ple_post_norm", "w_q", "w_k", "w_v", "w_o",
                                  "w_gate", "w_up", "w_down", "ple_input_gate", "ple_layer_projection")]


def _declare(L):
    sz, i32, i64, u32, u64, u16, vp = C.c_size_t, C.c_int32, C.c_int64, C.c_uint32, C.c_uint64, C.c_uint16, C.c_void_p
    sig = {
        "dn_rshift_round_ties_even": (i64, [i64, u32]),
        "dn_requantize": (i32, [i64]),
        "dn_add_sat": (i32, [i32, i32]), "dn_sub_sat": (i32, [i32, i32]), "dn_mul_sat": (i32, [i32, i32]),
        "dn_acc_add_sat": (i64, [i64, i64]),
        "dn_div_act": (i32, [i32, i32]), "dn_div_acc": (i64, [i64, i64]),
        "dn_div_acc_by_u32": (i64, [i64, u32]), "dn_acc_mul": (i64, [i64, i64]),
        "dn_inv_sqrt_acc": (i32, [i64]),
        "dn_rms_norm_scale": (i32, [i32p, sz, i64]),
        "dn_rms_norm": (None, [i32p, i32p, sz, i64]),
        "dn_value_rms_norm": (None, [i32p, sz, i64]),
        "dn_argmax_first": (sz, [i32p, sz]),
        "dn_softmax_exp_term": (i64, [i64]),
        "dn_attention_softmax": (None, [i32p, sz, i64p, i32p]),
        "dn_tanh_act": (i32, [i32]), "dn_softcap_act": (i32, [i32, i32]), "dn_gelu": (i32, [i32]),
        "dn_nth_root_acc": (i64, [i64, u32]), "dn_pow_acc_u32": (i64, [i64, u32]),
        "dn_rope_frequency_step": (i64, [i64, sz]),
        "dn_sin_cos_acc": (None, [i64, C.POINTER(i32), C.POINTER(i32)]),
        "dn_rope_rotate_pairs": (None, [i32p, sz, sz, sz, i64, sz]),
        "dn_dot_bits": (i32, [i32p, i32p, sz]),
        "dn_scale_q24": (C.c_int, [u16, C.POINTER(i64)]),
        "dn_q8_dot_row": (C.c_int, [i32p, u8p, sz, C.POINTER(i32)]),
        "dn_q8_dequantize_row": (C.c_int, [u8p, sz, i32p]),
        "dn_exp_neg_q32": (u64, [u64]), "dn_sigmoid_q32": (u64, [i32]), "dn_silu": (i32, [i32]),
        "dn_sin_cos_q30": (None, [i64, C.POINTER(i64), C.POINTER(i64)]),
        "dn_rotate_consecutive_pairs": (None, [i32p, sz, i64p, sz, u32]),
        "dn_scaled_score": (i32, [i32p, i32p, sz, u32]),
        "dn_attention_scale_q32": (u32, [u32]),
        "dn_yarn_inverse_frequencies": (C.c_int, [u64, u32, u32, u32, u32, i64p]),
        "dn_f32_to_act_bits": (i32, [C.c_float]), "dn_f32_to_acc_bits": (i64, [C.c_float]),
        "orc_linear_q8": (C.c_int, [i32p, sz, sz, u8p, sz, i32p, C.c_int]),
        "orc_linear_i32": (C.c_int, [i32p, sz, sz, i32p, sz, i32p, C.c_int]),
        "orc_mistral_layer_forward": (C.c_int, [C.POINTER(MistralLayerC), i32p, sz, u32, i32p, i32p, i32p, C.c_int]),
        "orc_gemma_layer_forward": (C.c_int, [C.POINTER(GemmaLayerC), i32p, sz, u32, i32p, i32p, i32p, i32p,
                                              i32p, i32p, C.c_int]),
        "orc_gemma_ple_prepare": (C.c_int, [i32p, sz, i32p, sz, i32, i32p, i64, u8p, sz, i32, i32, i32p]),
        "orc_head_logits": (C.c_int, [i32p, sz, i32p, i64, i32, u8p, sz, i32p, C.c_int]),
        "orc_embedding_row": (C.c_int, [u8p, sz, C.c_int, i32, i32p]),
        "orc_silu_many": (C.c_int, [i32p, sz, i32p, C.c_int]),
        "orc_mistral_layer_rows": (C.c_int, [C.POINTER(MistralLayerC), i32p, sz, u32, i32p, i32p, u32p, sz, i32p,
                                             C.c_int]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def _ptr(a) -> int:
    return a.ctypes.data


def _check(rc: int, what: str):
    if rc != 0:
        raise ValueError(f"oracle {what} failed with code {rc}")


# ------------------------------------------------------------ small wrappers

def q8_dot_row(act, row) -> int:
    act, row = _c(act, np.int32), _c(row, np.uint8)
    out = C.c_int32()
    _check(lib().dn_q8_dot_row(act, row, act.size, C.byref(out)), "q8 dot_row")
    return out.value


def linear_q8(inp, w, threads: int = 0) -> np.ndarray:
    """tokens x rows products of a Q8_0 matrix (raw bytes [rows, cols/32*34])."""
    inp = _c(np.atleast_2d(inp), np.int32)
    w = _c(w, np.uint8)
    tokens, cols = inp.shape
    rows = w.shape[0]
    out = np.empty((tokens, rows), dtype=np.int32)
    _check(lib().orc_linear_q8(inp, tokens, cols, w, rows, out, threads or default_threads()), "linear_q8")
    return out


def linear_i32(inp, w, threads: int = 0) -> np.ndarray:
    inp = _c(np.atleast_2d(inp), np.int32)
    w = _c(w, np.int32)
    out = np.empty((inp.shape[0], w.shape[0]), dtype=np.int32)
    _check(lib().orc_linear_i32(inp, inp.shape[0], inp.shape[1], w, w.shape[0], out, threads or default_threads()),
           "linear_i32")
    return out


def silu_many(x, threads: int = 0) -> np.ndarray:
    """mistral.rs:72-77 silu of every value."""
    x = _c(x, np.int32).reshape(-1)
    out = np.empty_like(x)
    _check(lib().orc_silu_many(x, x.size, out, threads or default_threads()), "silu")
    return out


def rms_norm(v, w, eps: int) -> np.ndarray:
    v = _c(v, np.int32).copy()
    lib().dn_rms_norm(v, _c(w, np.int32), v.size, eps)
    return v


def attention_softmax(logits) -> np.ndarray:
    logits = _c(logits, np.int32)
    scratch = np.empty(logits.size, dtype=np.int64)
    w = np.empty(logits.size, dtype=np.int32)
    lib().dn_attention_softmax(logits, logits.size, scratch, w)
    return w


def rope_rotate_pairs(v, rotary_dim, freq_base_dim, base, position) -> np.ndarray:
    v = _c(v, np.int32).copy()
    lib().dn_rope_rotate_pairs(v, v.size, rotary_dim, freq_base_dim, base, position)
    return v


def rotate_consecutive_pairs(v, inv_freq, position) -> np.ndarray:
    v = _c(v, np.int32).copy()
    f = _c(inv_freq, np.int64)
    lib().dn_rotate_consecutive_pairs(v, v.size, f, f.size, position)
    return v


def sin_cos_acc(angle: int):
    c, s = C.c_int32(), C.c_int32()
    lib().dn_sin_cos_acc(angle, C.byref(c), C.byref(s))
    return c.value, s.value


def sin_cos_q30(angle: int):
    s, c = C.c_int64(), C.c_int64()
    lib().dn_sin_cos_q30(angle, C.byref(s), C.byref(c))
    return s.value, c.value


def yarn_inverse_frequencies(base, pairs, factor, low, high):
    out = np.empty(max(pairs, 1), dtype=np.int64)
    rc = lib().dn_yarn_inverse_frequencies(base, pairs, factor, low, high, out)
    return None if rc else [int(x) for x in out[:pairs]]


# ------------------------------------------------------------ token loop


class OracleRun:
    """The reference's direct token loop over a model (iris_amd.model.Model
    duck type: family, shape, q8()/values()/layer_name()/... accessors)."""

    def __init__(self, model, max_positions: int, threads: int = 0):
        self.m = model
        self.threads = threads or default_threads()
        self.max_positions = max_positions
        self.keep = []  # numpy arrays the C structs point into
        s = model.shape
        self.layers = []
        self.k_cache, self.v_cache = [], []
        for layer in range(model.num_layers):
            hd = model.head_dim_at(layer)
            kvw = s.num_key_value_heads * hd
            self.k_cache.append(np.zeros((max_positions, kvw), dtype=np.int32))
            self.v_cache.append(np.zeros((max_positions, kvw), dtype=np.int32))
            self.layers.append(self._mistral_layer(layer) if model.family == "mistral-dense"
                               else self._gemma_layer(layer))
        self.position = 0
        self.last_row = None

    def _hold(self, a, dtype):
        a = _c(a, dtype)
        self.keep.append(a)
        return _ptr(a)

    def _mistral_layer(self, layer):
        m, s = self.m, self.m.shape
        L = MistralLayerC()
        L.hidden, L.ffn = s.hidden_size, s.intermediate_size
        L.heads, L.kv_heads, L.head_dim = s.num_attention_heads, s.num_key_value_heads, s.head_dim
        L.norm_eps, L.attention_scale_q32 = s.norm_eps, s.attention_scale_q32
        L.inv_freq = self._hold(np.array(s.rope_inverse_frequencies, dtype=np.int64), np.int64)
        L.max_positions = s.max_positions
        L.norm_attention = self._hold(m.values(m.layer_name(layer, "input_layernorm.weight")), np.int32)
        L.norm_feed_forward = self._hold(m.values(m.layer_name(layer, "pre_feedforward_layernorm.weight")), np.int32)
        for f, n in [("w_q", "self_attn.q_proj.weight"), ("w_k", "self_attn.k_proj.weight"),
                     ("w_v", "self_attn.v_proj.weight"), ("w_o", "self_attn.o_proj.weight"),
                     ("w_gate", "mlp.gate_proj.weight"), ("w_up", "mlp.up_proj.weight"),
                     ("w_down", "mlp.down_proj.weight")]:
            setattr(L, f, self._hold(m.q8(m.layer_name(layer, n)), np.uint8))
        return L

    def _gemma_layer(self, layer):
        m, s = self.m, self.m.shape
        L = GemmaLayerC()
        hd = m.head_dim_at(layer)
        base, rotary, fbd = m.rope_at(layer)
        L.hidden, L.ffn = s.hidden_size, m.ffn_size(layer)
        L.heads, L.kv_heads, L.head_dim = s.num_attention_heads, s.num_key_value_heads, hd
        L.ple_width = s.hidden_size_per_layer_input
        L.sliding_window = m.sliding_window_at(layer)
        L.layer_scalar = m.layer_scalar(layer)
        L.norm_eps, L.rope_base, L.rotary_dim, L.rope_freq_base_dim = s.norm_eps, base, rotary, fbd
        for f, n in [("norm_input", "input_layernorm.weight"), ("norm_post_attn", "post_attention_layernorm.weight"),
                     ("norm_pre_ffw", "pre_feedforward_layernorm.weight"),
                     ("norm_post_ffw", "post_feedforward_layernorm.weight"),
                     ("q_norm", "self_attn.q_norm.weight"), ("k_norm", "self_attn.k_norm.weight"),
                     ("ple_post_norm", "post_per_layer_input_norm.weight"),
                     ("ple_input_gate", "per_layer_input_gate.weight"),
                     ("ple_layer_projection", "per_layer_projection.weight")]:
            setattr(L, f, self._hold(m.values(m.layer_name(layer, n)), np.int32))
        for f, n in [("w_q", "self_attn.q_proj.weight"), ("w_k", "self_attn.k_proj.weight"),
                     ("w_v", "self_attn.v_proj.weight"), ("w_o", "self_attn.o_proj.weight"),
                     ("w_gate", "mlp.gate_proj.weight"), ("w_up", "mlp.up_proj.weight"),
                     ("w_down", "mlp.down_proj.weight")]:
            setattr(L, f, self._hold(m.q8(m.layer_name(layer, n)), np.uint8))
        return L

    # view_kernels.rs:14-57 / model.rs:316-330
    def embed(self, ids) -> np.ndarray:
        m = self.m
        H = m.hidden
        table = m.q8(m.embedding_name())
        scaled = m.family == "gemma-dense"  # only gemma-dense scales its embeddings
        scale = m.shape.embedding_scale if scaled else 0
        out = np.empty((len(ids), H), dtype=np.int32)
        for i, t in enumerate(ids):
            row = np.empty(H, dtype=np.int32)
            _check(lib().orc_embedding_row(_c(table[int(t)], np.uint8), H, int(scaled), scale, row), "embedding")
            out[i] = row
        return out

    def _ple_rows(self, layer, ids, seed_rows) -> np.ndarray:
        m, s = self.m, self.m.shape
        P, H = s.hidden_size_per_layer_input, s.hidden_size
        proj = _c(m.values("model.language_model.per_layer_model_projection.weight")
                  .reshape(-1, H)[layer * P:(layer + 1) * P], np.int32)
        norm = _c(m.values("model.language_model.per_layer_projection_norm.weight"), np.int32)
        table = m.q8("model.language_model.embed_tokens_per_layer.weight")
        out = np.empty((len(ids), P), dtype=np.int32)
        for i, t in enumerate(ids):
            row = np.empty(P, dtype=np.int32)
            _check(lib().orc_gemma_ple_prepare(_c(seed_rows[i], np.int32), H, proj, P, s.ple_projection_scalar,
                                               norm, s.norm_eps, _c(table[int(t)], np.uint8), layer * P,
                                               s.ple_embedding_scale, s.ple_input_scale, row), "ple prepare")
            out[i] = row
        return out

    def layer_pass(self, layer: int, x: np.ndarray, start: int, ids=None, seed_rows=None) -> np.ndarray:
        """One layer over rows at absolute positions start..start+len(x)."""
        x = _c(x, np.int32)
        out = np.empty_like(x)
        if self.m.family == "mistral-dense":
            _check(lib().orc_mistral_layer_forward(C.byref(self.layers[layer]), x, x.shape[0], start,
                                                   self.k_cache[layer], self.v_cache[layer], out,
                                                   self.threads), f"mistral layer {layer}")
        else:
            ple = self._ple_rows(layer, ids, seed_rows)
            donor = self.m.kv_donor_layer(layer)
            src = layer if donor < 0 else donor
            _check(lib().orc_gemma_layer_forward(C.byref(self.layers[layer]), x, x.shape[0], start,
                                                 self.k_cache[layer], self.v_cache[layer], self.k_cache[src],
                                                 self.v_cache[src], ple, out, self.threads),
                   f"gemma layer {layer}")
        return out

    def mistral_layer_rows(self, layer: int, x: np.ndarray, start: int, sel) -> np.ndarray:
        """One mistral-dense layer over rows at positions start..start+len(x):
        every row's keys and values into this run's caches, the layer output
        only for the row indices in ``sel`` ([len(sel), hidden])."""
        x = _c(x, np.int32)
        sel = _c(sel, np.uint32)
        out = np.empty((sel.size, x.shape[1]), dtype=np.int32)
        _check(lib().orc_mistral_layer_rows(C.byref(self.layers[layer]), x, x.shape[0], start, self.k_cache[layer],
                                            self.v_cache[layer], sel, sel.size, out, self.threads),
               f"mistral layer {layer} rows")
        return out

    def pass_rows(self, ids, start: int, keep_layers: bool = False):
        """Embed `ids` at `start`, run every layer; returns (final rows,
        per-layer outputs if asked)."""
        seed = self.embed(ids)
        cur = seed
        outs = []
        for layer in range(self.m.num_layers):
            cur = self.layer_pass(layer, cur, start, ids, seed)
            if keep_layers:
                outs.append(cur.copy())
        return cur, outs

    def logits(self, last_row) -> np.ndarray:
        m = self.m
        head = _c(m.q8(m.head_name()), np.uint8)
        out = np.empty(m.vocab, dtype=np.int32)
        _check(lib().orc_head_logits(_c(last_row, np.int32), m.hidden, _c(m.final_norm(), np.int32),
                                     m.shape.norm_eps, m.head_softcap(), head, m.vocab, out, self.threads), "head")
        return out

    def generate(self, prompt_ids, tokens: int, keep_logits: bool = False):
        """executor.rs:143-185: returns (token ids, list of logits per selection)."""
        rows, _ = self.pass_rows(prompt_ids, 0)
        position = len(prompt_ids)
        logits = self.logits(rows[-1])
        out, all_logits = [], []
        for t in range(tokens):
            if keep_logits:
                all_logits.append(logits.copy())
            tok = int(np.argmax(logits))  # numpy argmax returns the first maximum
            out.append(tok)
            if tok in self.m.eos_token_ids or t + 1 == tokens:
                break
            rows, _ = self.pass_rows([tok], position)
            position += 1
            logits = self.logits(rows[-1])
        return out, all_logits
