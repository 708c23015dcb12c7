"""DETWGT v3: the reference's weight-file format, read and written with numpy.

Layout (crates/model/detwgt/src/mmap.rs:9-18, parse_directory :462-529):
``b"DNWGTV0\\0"``, u32 version (2 or 3), u32 det-num spec (1), u64 tensor
count, then per tensor: u32 name length, name bytes, u32 rank, u64 dims[rank],
u64 element count, u32 element width, u64 payload length, u64 max row mass,
zero padding to a 64-byte boundary, payload. Element width 16 or 32 means
little-endian signed Q16.16 values (16-bit ones are sign-extended); width 8
means Q8_0 rows of 34-byte blocks (an f16 scale and 32 signed bytes).
"""
from __future__ import annotations

import math
import struct
from dataclasses import dataclass

import numpy as np

MAGIC = b"DNWGTV0\0"
VERSION = 3
SPEC = 1
ALIGN = 64
Q8_0_WIDTH = 8
BLOCK = 32
BLOCK_BYTES = 34


@dataclass
class Tensor:
    name: str
    dims: tuple
    width: int
    payload: object  # bytes or a view of a mapping
    offset: int = 0  # of the payload in the artifact

    def values(self) -> np.ndarray:
        """Q16.16 values as int32 (widths 16 and 32)."""
        if self.width == 32:
            return np.frombuffer(self.payload, dtype="<i4").astype(np.int32)
        if self.width == 16:
            return np.frombuffer(self.payload, dtype="<i2").astype(np.int32)
        raise ValueError(f"tensor '{self.name}' holds Q8_0 blocks, not Q16.16 values")

    def q8(self) -> np.ndarray:
        """Raw Q8_0 bytes as uint8 [rows, cols/32*34]."""
        if self.width != Q8_0_WIDTH:
            raise ValueError(f"tensor '{self.name}' is not Q8_0")
        cols = self.dims[-1]
        rows = math.prod(self.dims) // cols
        return np.frombuffer(self.payload, dtype=np.uint8).reshape(rows, cols // BLOCK * BLOCK_BYTES)


def scale_q24(bits: np.ndarray) -> np.ndarray:
    """Exact Q.24 value of f16 scale bits (crates/det-num/src/q8.rs:27-42);
    raises on inf/NaN."""
    bits = np.asarray(bits, dtype=np.int64)
    exponent = (bits >> 10) & 0x1F
    if np.any(exponent == 0x1F):
        raise ValueError("Q8_0 block scale is not finite")
    mantissa = bits & 0x3FF
    mag = np.where(exponent == 0, mantissa, (1024 + mantissa) << np.maximum(exponent - 1, 0))
    return np.where(bits & 0x8000, -mag, mag)


def _rte_shift(value: np.ndarray, shift: int) -> np.ndarray:
    floor = value >> shift
    rem = value - (floor << shift)
    half = 1 << (shift - 1)
    return np.where((rem > half) | ((rem == half) & ((floor & 1) == 1)), floor + 1, floor)


def q8_row_mass(data: np.ndarray) -> int:
    """Largest row sum of |dequantized value| in Q16.16 (the writer's
    ``max_row_mass``; the reference computes it the same way in its bundle
    generators)."""
    rows = data.shape[0]
    blocks = data.reshape(rows, -1, BLOCK_BYTES)
    bits = blocks[:, :, 0].astype(np.int64) | (blocks[:, :, 1].astype(np.int64) << 8)
    scale = scale_q24(bits)
    q = blocks[:, :, 2:].view(np.int8).astype(np.int64)
    vals = _rte_shift(q * scale[:, :, None], 8)
    return int(np.abs(vals).sum(axis=(1, 2)).max()) if rows else 0


def write(tensors) -> bytes:
    """Serialise (name, dims, width, data) tuples; data is a list/array of
    ints for widths 16/32 and raw bytes for Q8_0."""
    out = bytearray(MAGIC + struct.pack("<IIQ", VERSION, SPEC, len(tensors)))
    for name, dims, width, data in tensors:
        nb = name.encode()
        row_width = dims[-1]
        if width == Q8_0_WIDTH:
            payload = bytes(data)
            arr = np.frombuffer(payload, dtype=np.uint8).reshape(-1, row_width // BLOCK * BLOCK_BYTES)
            mass = q8_row_mass(arr)
        else:
            vals = np.asarray(data, dtype=np.int64)
            mass = int(np.abs(vals.reshape(-1, row_width)).sum(axis=1).max())
            payload = vals.astype("<i4" if width == 32 else "<i2").tobytes()
        out += struct.pack("<I", len(nb)) + nb + struct.pack("<I", len(dims))
        out += struct.pack("<" + "Q" * len(dims), *dims)
        out += struct.pack("<QIQQ", math.prod(dims), width, len(payload), mass)
        out += b"\0" * (-len(out) % ALIGN)
        out += payload
    return bytes(out)


def read(buf) -> dict:
    """Parse a DETWGT v2/v3 artifact into {name: Tensor}, with the reader's
    checks (crates/model/detwgt/src/mmap.rs:462-529). ``buf`` is bytes or
    any buffer (a mapping): payloads are views into it, not copies."""
    mv = memoryview(buf)
    n = len(mv)
    off = 0

    def take(k):
        nonlocal off
        if off + k > n:
            raise ValueError("detwgt artifact is truncated")
        s = mv[off:off + k]
        off += k
        return s

    if bytes(take(8)) != MAGIC:
        raise ValueError("not a detwgt artifact")
    version, spec, count = struct.unpack("<IIQ", take(16))
    if not 2 <= version <= VERSION:
        raise ValueError(f"detwgt v{version} is not supported")
    if spec != SPEC:
        raise ValueError(f"unsupported det_num spec version {spec}")
    tensors = {}
    for _ in range(count):
        (nlen,) = struct.unpack("<I", take(4))
        name = bytes(take(nlen)).decode()
        (rank,) = struct.unpack("<I", take(4))
        dims = struct.unpack("<" + "Q" * rank, take(8 * rank))
        elements, width, plen, _mass = struct.unpack("<QIQQ", take(28))
        if elements != math.prod(dims):
            raise ValueError(f"tensor '{name}' element count does not match its shape")
        if width in (16, 32):
            expected = elements * (width // 8)
        elif width == Q8_0_WIDTH and version >= 3:
            cols = dims[-1] if dims else 0
            if cols == 0 or cols % BLOCK:
                raise ValueError(f"Q8_0 tensor '{name}' rows are not whole blocks")
            expected = elements // cols * (cols // BLOCK * BLOCK_BYTES)
        else:
            raise ValueError(f"tensor '{name}' has element width {width}")
        if plen != expected:
            raise ValueError(f"tensor '{name}' payload length does not match its width")
        off += -off % ALIGN
        if off > n:
            raise ValueError("detwgt artifact is truncated")
        at = off
        payload = take(plen)
        if name in tensors:
            raise ValueError(f"duplicate tensor '{name}' in artifact")
        tensors[name] = Tensor(name, tuple(dims), width, payload, at)
    if off != n:
        raise ValueError("trailing bytes after the last tensor payload")
    return tensors


class MappedDetwgt:
    """A DETWGT file mapped read-only (MmapDetwgt::open,
    crates/model/detwgt/src/mmap.rs): the directory is parsed with read()'s
    checks and every tensor's payload is a view of the mapping, so the
    weights are paged in from the file as they are used, never copied
    whole. ``key(name)`` names a tensor's bytes for as long as the mapping
    lives (the reference's Q8Key::mapped(mapping, offset),
    crates/inference/kernels/src/tensor.rs:90-108)."""

    _next_mapping = 1

    def __init__(self, path: str):
        import mmap
        self.path = path
        self._file = open(path, "rb")
        try:
            self._map = mmap.mmap(self._file.fileno(), 0, access=mmap.ACCESS_READ)
        except ValueError:  # an empty file cannot be mapped
            self._file.close()
            raise ValueError("not a detwgt artifact")
        self.mapping = MappedDetwgt._next_mapping
        MappedDetwgt._next_mapping += 1
        self.tensors = read(memoryview(self._map))

    def key(self, name: str) -> tuple:
        return (self.mapping, self.tensors[name].offset)

    def close(self):
        self.tensors = {}
        if self._map is not None:
            try:
                self._map.close()
            except BufferError:
                pass  # views still alive keep the mapping until they go
            self._map = None
        self._file.close()

