"""GPU parity of the one-token product that reads its row as digit planes
(the decode O and down products), through the C ABI, against the oracle.

iris_time_bcast_product forms the row's planes once, then runs the product
from them (one iteration here). Shapes cover one to four k slices per group
(with the last group's four tiles partly past the rows), block counts that
leave a ragged last run of four, and the smallest row the product takes
(256 values: one block per wave). Activation regimes cover each digit
count: 1, 2-3 (the unrolled path), 4 and 5 (the compact path, i32::MIN and
i32::MAX included), and a row whose waves need different counts.
"""
import ctypes as C

import numpy as np
import pytest

from iris_amd import native
from iris_amd.tensor import Q8Matrix
from oracle import cpu

pytestmark = pytest.mark.gpu


def row_scale_matrix(rng, rows, cols, max_exponent):
    """Every weight byte; one finite f16 scale of either sign per row."""
    nb = cols // 32
    v = rng.integers(0, 1 << 62, rows, dtype=np.int64)
    bits = ((v & 1) << 15) | (((v >> 20) % (max_exponent + 1)) << 10) | ((v >> 4) & 0x3FF)
    raw = np.empty((rows, nb, 34), np.uint8)
    raw[:, :, 0] = (bits & 0xFF)[:, None]
    raw[:, :, 1] = ((bits >> 8) & 0xFF)[:, None]
    raw[:, :, 2:] = rng.integers(0, 256, (rows, nb, 32))
    return raw.reshape(rows, -1)


def activations(rng, cols, kind):
    if kind == "one_digit":
        return rng.integers(-128, 128, (1, cols)).astype(np.int32)
    if kind == "three_digits":
        return rng.integers(-(1 << 23), 1 << 23, (1, cols)).astype(np.int32)
    if kind == "four_digits":
        return rng.integers(-(1 << 31), 1 << 31, (1, cols), dtype=np.int64).astype(np.int32) >> 1
    if kind == "extremes":
        x = rng.integers(-(1 << 31), 1 << 31, (1, cols), dtype=np.int64).astype(np.int32)
        x[0, ::61] = 2 ** 31 - 1
        x[0, 1::61] = -2 ** 31
        return x
    # mixed: small values with a few 5-digit ones, so waves take both paths
    x = rng.integers(-(1 << 15), 1 << 15, (1, cols)).astype(np.int32)
    x[0, ::331] = -2 ** 31
    return x


@pytest.fixture(scope="module", autouse=True)
def device():
    native.check(native.lib().q8gpu_init(), "q8gpu_init")


@pytest.mark.parametrize("rows,cols", [(1000, 256), (200, 4160), (64, 8224), (4100, 1024), (2048, 2048),
                                       (1000, 4096), (96, 14336)])
@pytest.mark.parametrize("kind", ["one_digit", "three_digits", "four_digits", "extremes", "mixed"])
def test_product_from_digit_planes_equals_the_oracle(rows, cols, kind):
    print(f"shape {rows}x{cols} activations {kind}", flush=True)
    rng = np.random.default_rng(rows * 7919 + cols * 31 + len(kind))
    raw = row_scale_matrix(rng, rows, cols, 24)
    x = activations(rng, cols, kind)
    m = Q8Matrix.from_bytes(raw, rows, cols)
    dx = native.DeviceBuffer.from_array(x)
    dout = native.DeviceBuffer(rows * 4)
    arr = (C.c_void_p * 1)(m.handle.value)
    ms = C.c_double()
    native.check(native.lib().iris_time_bcast_product(arr, 1, dx.ptr, dout.ptr, 1, C.byref(ms)), "bcast product")
    got = dout.to_array(np.int32, (1, rows))
    want = cpu.linear_q8(x, raw)
    m.free()
    assert np.array_equal(got, want)


def test_refuses_what_it_does_not_take():
    rng = np.random.default_rng(5)
    x = native.DeviceBuffer.from_array(activations(rng, 128, "one_digit"))
    out = native.DeviceBuffer(64 * 4)
    ms = C.c_double()
    m = Q8Matrix.from_bytes(row_scale_matrix(rng, 64, 128, 10), 64, 128)  # under 256 values: one block per wave
    arr = (C.c_void_p * 1)(m.handle.value)
    assert native.lib().iris_time_bcast_product(arr, 1, x.ptr, out.ptr, 1, C.byref(ms)) == -1
    m.free()
