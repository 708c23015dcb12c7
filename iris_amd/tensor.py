"""Device-resident Q8_0 matrices and the product dispatch.

Mirrors the reference's product surface (crates/inference/kernels/src/tensor.rs):
``Q8Matrix`` stands for a ``MatrixSource`` whose ``q8_source`` is on the GPU,
and ``linear_slab_from_source(input, matrix)`` returns ``out[t][r] =
q8::dot_row(input[t], W[r])`` (tensor.rs:437-520) computed by libiris_hip.
Errors follow the reference's: a width mismatch raises, a non-finite block
scale raises (q8.rs:45-47), no tokens gives an empty result.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import native

SCALE_MODES = {0: "row", 1: "f16", 2: "i64"}


class Q8Matrix:
    """A Q8_0 matrix uploaded to the GPU from its committed bytes."""

    def __init__(self, handle, rows: int, cols: int):
        self._h = handle
        self.rows, self.cols = rows, cols

    @classmethod
    def from_bytes(cls, raw: np.ndarray, rows: int, cols: int) -> "Q8Matrix":
        """Raw Q8_0 rows (rows x cols/32 blocks of 34 bytes)."""
        if cols <= 0 or cols % 32:
            raise ValueError(f"rows of {cols} values are not whole Q8_0 blocks")
        raw = np.ascontiguousarray(raw, dtype=np.uint8).reshape(-1)
        if raw.size != rows * (cols // 32) * 34:
            raise ValueError(f"{raw.size} bytes, expected {rows * (cols // 32) * 34} ({rows} x {cols} Q8_0)")
        h = C.c_void_p()
        native.check(native.lib().q8gpu_upload_q8_0(raw, rows, cols, C.byref(h)), "Q8_0 upload")
        return cls(h, rows, cols)

    @classmethod
    def from_weights_and_scales(cls, weights: np.ndarray, scales: np.ndarray) -> "Q8Matrix":
        """The reference device ABI's input: int8 [rows, cols] and i64 Q.24
        scales [rows, cols/32] (q8_product.cu:148-172)."""
        w = np.ascontiguousarray(weights, dtype=np.int8)
        s = np.ascontiguousarray(scales, dtype=np.int64)
        rows, cols = w.shape
        h = C.c_void_p()
        native.check(native.lib().q8gpu_upload(w.reshape(-1), s.reshape(-1), rows, cols, C.byref(h)), "upload")
        return cls(h, rows, cols)

    @property
    def handle(self):
        return self._h

    def prepare_matrix_cores(self):
        """Fold a per-block scale matrix for the int8 matrix cores (one to
        six more bytes per weight, by how far a row's scales spread; nothing
        for a row-scale matrix): its multi-token products then run there."""
        native.check(native.lib().q8gpu_prepare_matrix_cores(self._h, None), "prepare matrix cores")

    def info(self):
        r, c, mode, b = C.c_uint32(), C.c_uint32(), C.c_int(), C.c_uint64()
        native.check(native.lib().q8gpu_matrix_info(self._h, C.byref(r), C.byref(c), C.byref(mode), C.byref(b)),
                     "matrix info")
        return {"rows": r.value, "cols": c.value, "scale_mode": SCALE_MODES[mode.value], "bytes": b.value}

    def free(self):
        if self._h:
            native.lib().q8gpu_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class UploadCache:
    """Device copies of Q8_0 matrices by the key that names their bytes (the
    reference's Q8Key, crates/inference/kernels/src/tensor.rs:90-108: a
    mapped tensor's (mapping, offset), or a unique key), least recently used
    first out once the held bytes would pass ``budget`` (the reference's
    device cache, crates/inference/kernels/src/gpu.rs:176-208).

    As there, each entry counts rows * cols + blocks * 8 bytes, fixed when it
    is inserted (gpu.rs:171-173), and the entries to evict go before the
    upload. An evicted matrix leaves the cache; its device memory is released
    when the last holder of the returned Q8Matrix lets it go, so a matrix a
    caller still holds stays valid."""

    def __init__(self, budget: int = 64 << 30):
        from collections import OrderedDict
        self.budget = budget
        self.held = 0
        self._items = OrderedDict()  # key -> (matrix, counted bytes)
        self.uploads = 0

    @staticmethod
    def counted_bytes(rows: int, cols: int) -> int:
        return rows * cols + rows * (cols // 32) * 8

    def get(self, key, raw: np.ndarray, rows: int, cols: int) -> Q8Matrix:
        hit = self._items.get(key)
        if hit is not None:
            self._items.move_to_end(key)
            return hit[0]
        size = self.counted_bytes(rows, cols)
        while self._items and self.held + size > self.budget:
            _, (_, old_size) = self._items.popitem(last=False)
            self.held -= old_size
        m = Q8Matrix.from_bytes(raw, rows, cols)
        self.uploads += 1
        self._items[key] = (m, size)
        self.held += size
        return m

    def __len__(self):
        return len(self._items)

    def __contains__(self, key):
        return key in self._items

    def clear(self):
        self._items.clear()
        self.held = 0


def linear_slab_from_source(inp: np.ndarray, matrix: Q8Matrix) -> np.ndarray:
    """out[t][r] = dot_row(inp[t], W[r]) for every token row of ``inp``."""
    inp = np.ascontiguousarray(np.atleast_2d(inp), dtype=np.int32)
    if inp.shape[1] != matrix.cols:
        raise ValueError(f"deterministic linear input row 0 has width {inp.shape[1]}, expected {matrix.cols}")
    out = np.empty((inp.shape[0], matrix.rows), dtype=np.int32)
    if inp.shape[0] == 0:
        return out
    native.check(native.lib().q8gpu_product(matrix.handle, inp.reshape(-1), inp.shape[0], out.reshape(-1)),
                 "Q8_0 product")
    return out
