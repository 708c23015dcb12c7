"""The staged (teacher-forced) layer pass over ranges, on the GPU.

Host-side mirror of the reference's stage boundary: the ``ActivationRow``,
``KeyRow`` and ``ActivationSequence`` values a layer stage takes and
returns (raster-stages/prefill-range/src/input.rs:43-190), ``output_kv``
(crates/inference/kernels/src/prefill_range.rs:849-872), the one-layer stage
(``run_layer_stage``, crates/inference/kernels/src/mistral/stage.rs:172-226;
gemma-dense ``run_prefill_range_direct``, prefill_range.rs:82-172) and the
whole chain over one range. The rows and keys come from libiris_hip through
``direct.Session``; nothing here computes a value.

Rows and keys are little-endian int32 bytes, as the reference's pages are.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from . import native
from .direct import Session


@dataclass(frozen=True)
class ActivationRow:
    token_id: int
    values: bytes  # hidden x LE i32


@dataclass(frozen=True)
class KeyRow:
    position: int
    k: bytes  # kv_heads * head_dim x LE i32
    v: bytes


@dataclass
class ActivationSequence:
    rows: list
    kv: list
    start_position: int
    errors: list = field(default_factory=list)

    def values(self) -> np.ndarray:
        """The rows' values as an [n, hidden] int32 array."""
        if not self.rows:
            return np.zeros((0, 0), dtype=np.int32)
        return np.stack([np.frombuffer(r.values, dtype="<i4") for r in self.rows]).astype(np.int32)


def window_start(query_position: int, sliding_window: int) -> int:
    """First key position a query at ``query_position`` sees
    (prefill_range.rs:864-872): 0 for full attention."""
    if sliding_window == 0:
        return 0
    return max(0, query_position + 1 - sliding_window)


def output_kv(prior_keys, own_keys, start_position: int, sliding_window: int) -> list:
    """The keys a range hands to the next one (prefill_range.rs:849-862):
    what the window still holds of the inherited keys, then its own."""
    keep_from = window_start(start_position, sliding_window)
    return [k for k in prior_keys if k.position >= keep_from] + list(own_keys)


def key_rows(k: np.ndarray, v: np.ndarray, pos0: int) -> list:
    return [KeyRow(pos0 + i, np.ascontiguousarray(k[i], dtype="<i4").tobytes(),
                   np.ascontiguousarray(v[i], dtype="<i4").tobytes()) for i in range(k.shape[0])]


def _key_arrays(keys) -> tuple:
    k = np.stack([np.frombuffer(r.k, dtype="<i4") for r in keys]).astype(np.int32)
    v = np.stack([np.frombuffer(r.v, dtype="<i4") for r in keys]).astype(np.int32)
    return k, v


def _contiguous(keys) -> bool:
    return all(b.position == a.position + 1 for a, b in zip(keys, keys[1:]))


def _sliding_window(session: Session, layer: int) -> int:
    m = session.dm.model
    return m.sliding_window_at(layer) if m.family == "gemma-dense" else 0


def _carry(session: Session, layer: int, prior_keys) -> None:
    """Writes a layer's inherited keys into the session's cache; they must
    be consecutive positions, as the reference's coverage check requires
    (raster-stages/layer-mistral/src/lib.rs:889-940)."""
    if not prior_keys:
        return
    if not _contiguous(prior_keys):
        raise native.IrisError(-4, f"layer {layer} carried keys are not consecutive positions")
    k, v = _key_arrays(prior_keys)
    session.write_kv(layer, prior_keys[0].position, k, v)


def run_layer_stage(session: Session, layer: int, activations: ActivationSequence, prior_kv, ple_rows=None):
    """One layer over one range (mistral/stage.rs:172-226): the layer's rows
    for ``activations`` (the layer below's output) over ``prior_kv`` and the
    range's own keys; ``kv`` = the window's part of prior_kv ++ own keys. A
    range whose inherited keys do not cover what it attends to passes on no
    rows and carries the cache, with the reason in ``errors``, as the stage
    does."""
    start = activations.start_position
    window = _sliding_window(session, layer)
    try:
        _carry(session, layer, prior_kv)
        x = activations.values()
        out = session.layer_stage(layer, x, start, ple_rows)
    except native.IrisError as e:
        if e.code != -4:
            raise
        return ActivationSequence([], output_kv(prior_kv, [], start, window), start, [str(e)])
    k, v = session.read_kv(layer, start, out.shape[0])
    rows = [ActivationRow(r.token_id, np.ascontiguousarray(out[i], dtype="<i4").tobytes())
            for i, r in enumerate(activations.rows)]
    return ActivationSequence(rows, output_kv(prior_kv, key_rows(k, v, start), start, window), start)


def run_chain_range(session: Session, ids, start_position: int, prior_kv=None):
    """Every layer over one range of token ids at ``start_position`` (the
    chain's per-layer stages one after the other): a list with one
    ActivationSequence per layer. ``prior_kv[l]`` are layer l's inherited
    keys (None: the caches already hold them from this session's earlier
    ranges)."""
    ids = [int(t) for t in ids]
    if prior_kv is not None:
        for layer, keys in enumerate(prior_kv):
            _carry(session, layer, keys)
    rows, _ = session.layer_range(ids, start_position)
    out = []
    for layer in range(rows.shape[0]):
        k, v = session.read_kv(layer, start_position, len(ids))
        prior = prior_kv[layer] if prior_kv is not None else []
        window = _sliding_window(session, layer)
        seq_rows = [ActivationRow(t, np.ascontiguousarray(rows[layer][i], dtype="<i4").tobytes())
                    for i, t in enumerate(ids)]
        out.append(ActivationSequence(seq_rows, output_kv(prior, key_rows(k, v, start_position), start_position,
                                                          window), start_position))
    return out
