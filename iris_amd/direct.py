"""The deterministic token loop on the GPU, through libiris_hip's C ABI.

Host-side mirror of the reference's direct-infer surface
(crates/inference/direct/src/executor.rs:17-39 ``DirectInferenceExecutor``,
model.rs ``DirectInferenceModel``): a ``DeviceModel`` holds one model's
weights on the device, a ``Session`` holds a KV cache and runs greedy
generation (executor.rs:143-185) or the teacher-forced per-layer pass the
chain's layer stages compute (staged/src/routines/layer_mistral.rs:80-99).
Every number comes from the HIP library; nothing here computes on the CPU.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import numpy as np

from . import native
from .model import PREFIX, Model

FAMILY = {"mistral-dense": 0, "gemma-dense": 1}


class ModelDesc(C.Structure):
    _fields_ = [("family", C.c_int32), ("hidden", C.c_uint32), ("layers", C.c_uint32), ("heads", C.c_uint32),
                ("kv_heads", C.c_uint32), ("head_dim", C.c_uint32), ("ffn", C.c_uint32), ("vocab", C.c_uint32),
                ("norm_eps", C.c_int64), ("attention_scale_q32", C.c_uint32), ("max_positions", C.c_uint32),
                ("tied_head", C.c_int32), ("global_head_dim", C.c_uint32), ("ple_width", C.c_uint32),
                ("sliding_window", C.c_uint32), ("num_kv_shared_layers", C.c_uint32),
                ("rope_base_sliding", C.c_int64), ("rope_base_full", C.c_int64),
                ("partial_rotary_q16", C.c_int32), ("embedding_scale", C.c_int32),
                ("ple_embedding_scale", C.c_int32), ("ple_projection_scalar", C.c_int32),
                ("ple_input_scale", C.c_int32), ("final_logit_softcap", C.c_int32),
                ("layer_is_sliding", C.c_void_p)]


def _declare():
    L = native.lib()
    if getattr(L, "_iris_direct_declared", False):
        return L
    vp, u32, i32, u64 = C.c_void_p, C.c_uint32, C.c_int32, C.c_uint64
    pp = C.POINTER(C.c_void_p)
    sig = {
        "iris_model_create": (C.c_int, [C.POINTER(ModelDesc), pp]),
        "iris_model_set_tensor": (C.c_int, [vp, C.c_char_p, i32, vp, u64, u64]),
        "iris_model_finalize": (C.c_int, [vp]),
        "iris_model_free": (None, [vp]),
        "iris_model_device_bytes": (u64, [vp]),
        "iris_session_create": (C.c_int, [vp, u32, u32, pp]),
        "iris_session_free": (None, [vp]),
        "iris_session_generate": (C.c_int, [vp, vp, u32, u32, vp, u32, vp, C.POINTER(u32), vp, i32]),
        "iris_session_layer_pass": (C.c_int, [vp, vp, u32, vp, vp]),
        "iris_session_layer_range": (C.c_int, [vp, vp, u32, u32, vp, vp]),
        "iris_session_layer_stage": (C.c_int, [vp, u32, vp, u32, u32, vp, vp]),
        "iris_session_write_kv": (C.c_int, [vp, u32, u32, u32, vp, vp]),
        "iris_session_time_decode": (C.c_int, [vp, vp, u32, u32, C.POINTER(C.c_double), C.POINTER(C.c_double), vp]),
        "iris_session_time_decode_launches": (C.c_int, [vp, vp, u32, u32, C.c_int, C.POINTER(C.c_double),
                                                        C.POINTER(C.c_double), vp]),
        "iris_session_time_pass": (C.c_int, [vp, vp, u32, C.POINTER(C.c_double)]),
        "iris_session_read_kv": (C.c_int, [vp, u32, u32, u32, vp, vp]),
        "iris_sha256_bytes": (C.c_int, [vp, u64, vp]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    L._iris_direct_declared = True
    return L


def _desc(model: Model) -> ModelDesc:
    s = model.shape
    d = ModelDesc()
    d.family = FAMILY[model.family]
    d.hidden, d.layers = s.hidden_size, s.num_hidden_layers
    d.heads, d.kv_heads, d.head_dim = s.num_attention_heads, s.num_key_value_heads, s.head_dim
    d.vocab = s.vocab_size
    d.norm_eps = s.norm_eps
    d.tied_head = int(s.tied_head)
    if model.family == "mistral-dense":
        d.ffn = s.intermediate_size
        d.attention_scale_q32 = s.attention_scale_q32
        d.max_positions = s.max_positions
    else:
        d.ffn = model.ffn_size(0) if model.num_layers else 0
        d.global_head_dim = s.global_head_dim
        d.ple_width = s.hidden_size_per_layer_input
        d.sliding_window = s.sliding_window
        d.num_kv_shared_layers = s.num_kv_shared_layers
        d.rope_base_sliding, d.rope_base_full = s.rope_base_sliding, s.rope_base_full
        d.partial_rotary_q16 = s.full_partial_rotary_factor_q16
        d.embedding_scale, d.ple_embedding_scale = s.embedding_scale, s.ple_embedding_scale
        d.ple_projection_scalar, d.ple_input_scale = s.ple_projection_scalar, s.ple_input_scale
        d.final_logit_softcap = s.final_logit_softcap
        d.max_positions = 1 << 30
    return d


class DeviceModel:
    """A model's weights on the device (the reference's mmap'd
    DirectInferenceModel, crates/inference/direct/src/model.rs:167-233)."""

    def __init__(self, model: Model):
        L = _declare()
        self.model = model
        self.desc = _desc(model)
        self._sliding = None
        if model.family == "gemma-dense":
            self._sliding = (C.c_uint8 * model.num_layers)(*[int(model.is_sliding(i)) for i in range(model.num_layers)])
            self.desc.layer_is_sliding = C.cast(self._sliding, C.c_void_p)
        h = C.c_void_p()
        native.check(L.iris_model_create(C.byref(self.desc), C.byref(h)), "model create")
        self._h = h
        try:
            if model.family == "mistral-dense":
                f = np.ascontiguousarray(model.shape.rope_inverse_frequencies, dtype=np.int64)
                self._set("rope_inverse_frequencies", 64, f, 1, f.size)
            for name, t in model.tensors.items():
                if t.dtype == np.uint8:
                    cols = t.shape[1] // 34 * 32
                    self._set(name, 8, t, t.shape[0], cols)
                else:
                    a = np.ascontiguousarray(t, dtype=np.int32)
                    rows, cols = (a.shape[0], a.shape[1]) if a.ndim == 2 else (1, a.size)
                    self._set(name, 32, a, rows, cols)
            native.check(L.iris_model_finalize(self._h), "model finalize")
        except Exception:
            self.free()
            raise

    @classmethod
    def from_manifest(cls, manifest_path: str) -> "DeviceModel":
        """The model a verified manifest names (ModelManifest::load_verified,
        crates/inference/artifacts/src/direct.rs:135-177), its DETWGT mapped
        and uploaded tensor by tensor from the mapping
        (DirectInferenceModel::load, crates/inference/direct/src/model.rs:
        167-233). ``.manifest`` keeps the manifest."""
        from . import artifacts
        manifest, model, mapped = artifacts.load_model(manifest_path)
        try:
            dm = cls(model)
        finally:
            model.tensors = {}
            mapped.close()
        dm.manifest = manifest
        return dm

    def _set(self, name, width, arr, rows, cols):
        arr = np.ascontiguousarray(arr)
        native.check(native.lib().iris_model_set_tensor(self._h, name.encode(), width, arr.ctypes.data, rows, cols),
                     f"set tensor {name}")

    @property
    def handle(self):
        return self._h

    def device_bytes(self) -> int:
        return int(native.lib().iris_model_device_bytes(self._h))

    def free(self):
        if getattr(self, "_h", None):
            native.lib().iris_model_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


@dataclass
class GenerateResult:
    token_ids: list
    logits: np.ndarray | None  # [selections, vocab]
    # "eos" when the last selection is an EOS id, else "max_new_tokens"
    # (the reference's report field, crates/inference/direct/src/executor.rs:157-171)
    stop_reason: str = "max_new_tokens"

    @property
    def token_ids_sha256(self) -> str:
        """SHA-256 of the ids as compact JSON (``[2,0]``): the reference's
        generated_token_ids_sha256 (serde_json::to_vec of the id list)."""
        import hashlib
        return hashlib.sha256(("[" + ",".join(str(t) for t in self.token_ids) + "]").encode()).hexdigest()


class Session:
    """A KV cache of ``max_positions`` positions and passes of up to
    ``max_rows`` rows over a DeviceModel."""

    def __init__(self, dm: DeviceModel, max_positions: int, max_rows: int):
        L = _declare()
        self.dm = dm
        h = C.c_void_p()
        native.check(L.iris_session_create(dm.handle, max_positions, max_rows, C.byref(h)), "session create")
        self._h = h

    def generate(self, prompt_ids, tokens: int, keep_logits: bool = False, use_graph: bool = True) -> GenerateResult:
        prompt = np.ascontiguousarray(prompt_ids, dtype=np.int32)
        out = np.zeros(max(tokens, 1), dtype=np.int32)
        eos = np.ascontiguousarray(self.dm.model.eos_token_ids or [0], dtype=np.int32)
        logits = np.zeros((max(tokens, 1), self.dm.model.vocab), dtype=np.int32) if keep_logits else None
        count = C.c_uint32()
        native.check(native.lib().iris_session_generate(
            self._h, prompt.ctypes.data, prompt.size, tokens, eos.ctypes.data, len(self.dm.model.eos_token_ids),
            out.ctypes.data, C.byref(count), logits.ctypes.data if keep_logits else None, int(use_graph)),
            "generate")
        n = count.value
        ids = out[:n].tolist()
        eos = n > 0 and ids[-1] in self.dm.model.eos_token_ids
        return GenerateResult(ids, logits[:n] if keep_logits else None, "eos" if eos else "max_new_tokens")

    def layer_pass(self, ids, keep_rows: bool = True):
        """Teacher-forced pass: (rows [layers, n, hidden] or None, SHA-256 per layer)."""
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        m = self.dm.model
        rows = np.zeros((m.num_layers, ids.size, m.hidden), dtype=np.int32) if keep_rows else None
        hashes = np.zeros((m.num_layers, 32), dtype=np.uint8)
        native.check(native.lib().iris_session_layer_pass(self._h, ids.ctypes.data, ids.size,
                                                          rows.ctypes.data if keep_rows else None,
                                                          hashes.ctypes.data), "layer pass")
        return rows, [bytes(h).hex() for h in hashes]

    def layer_range(self, ids, start_position: int, keep_rows: bool = True):
        """The chain pass over one range at ``start_position`` over the keys
        the caches hold for the positions before it: (rows [layers, n,
        hidden] or None, SHA-256 per layer). Raises IrisError (IRIS_E_STATE)
        when a cache lacks a position the range needs."""
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        m = self.dm.model
        rows = np.zeros((m.num_layers, ids.size, m.hidden), dtype=np.int32) if keep_rows else None
        hashes = np.zeros((m.num_layers, 32), dtype=np.uint8)
        native.check(native.lib().iris_session_layer_range(self._h, ids.ctypes.data, ids.size, start_position,
                                                           rows.ctypes.data if keep_rows else None,
                                                           hashes.ctypes.data), "layer range")
        return rows, [bytes(h).hex() for h in hashes]

    def layer_stage(self, layer: int, in_rows, start_position: int, ple_rows=None):
        """One layer over one range: the layer's output rows [n, hidden] for
        input rows [n, hidden] at start_position.. (gemma-dense: with the
        layer's PLE rows [n, ple_width])."""
        x = np.ascontiguousarray(in_rows, dtype=np.int32)
        out = np.empty_like(x)
        ple = None if ple_rows is None else np.ascontiguousarray(ple_rows, dtype=np.int32)
        native.check(native.lib().iris_session_layer_stage(self._h, layer, x.ctypes.data, x.shape[0], start_position,
                                                           None if ple is None else ple.ctypes.data,
                                                           out.ctypes.data), f"layer {layer} stage")
        return out

    def write_kv(self, layer: int, pos0: int, k, v):
        """Carried keys into a layer's cache: rows [count, kv_heads*head_dim]
        of k and v for positions pos0.. (the reference's KeyRow k and v)."""
        k = np.ascontiguousarray(k, dtype=np.int32)
        v = np.ascontiguousarray(v, dtype=np.int32)
        if k.shape != v.shape or k.ndim != 2:
            raise ValueError("k and v must be [count, kv_width] arrays of one shape")
        native.check(native.lib().iris_session_write_kv(self._h, layer, pos0, k.shape[0], k.ctypes.data,
                                                        v.ctypes.data), "write kv")

    def time_decode(self, prompt_ids, steps: int, use_graph: bool = True):
        """(ms per decode token, prefill ms, generated ids) from HIP events;
        the decode passes as graph replays, or launch by launch."""
        prompt = np.ascontiguousarray(prompt_ids, dtype=np.int32)
        ms, pre = C.c_double(), C.c_double()
        toks = np.zeros(steps + 1, dtype=np.int32)
        native.check(native.lib().iris_session_time_decode_launches(self._h, prompt.ctypes.data, prompt.size, steps,
                                                                    int(use_graph), C.byref(ms), C.byref(pre),
                                                                    toks.ctypes.data),
                     "time decode")
        return ms.value, pre.value, toks.tolist()

    def read_kv(self, layer: int, pos0: int, count: int):
        """A layer's cached (k, v) rows of positions pos0..pos0+count, each
        [count, kv_heads*head_dim] int32 (the reference's KeyRow k and v)."""
        m = self.dm.model
        kvw = m.shape.num_key_value_heads * m.head_dim_at(layer)
        k = np.empty((count, kvw), dtype=np.int32)
        v = np.empty((count, kvw), dtype=np.int32)
        native.check(native.lib().iris_session_read_kv(self._h, layer, pos0, count, k.ctypes.data, v.ctypes.data),
                     "read kv")
        return k, v

    def time_pass(self, ids) -> float:
        """Milliseconds of one pass of every layer over ``ids`` (HIP events)."""
        ids = np.ascontiguousarray(ids, dtype=np.int32)
        ms = C.c_double()
        native.check(native.lib().iris_session_time_pass(self._h, ids.ctypes.data, ids.size, C.byref(ms)),
                     "time pass")
        return ms.value

    def free(self):
        if getattr(self, "_h", None):
            native.lib().iris_session_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def sha256(data: bytes) -> str:
    out = (C.c_uint8 * 32)()
    buf = np.frombuffer(data, dtype=np.uint8) if data else np.zeros(1, np.uint8)
    native.check(_declare().iris_sha256_bytes(buf.ctypes.data, len(data), out), "sha256")
    return bytes(out).hex()
