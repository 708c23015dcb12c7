"""The no-allocation product entry point against the work-space one.

q8gpu_product_device_noalloc keeps its work space in a device array of the
library instead of memory the caller brings. Its outputs must equal
q8gpu_product_device_ws's bit for bit: two calls in a row on one stream (the
second with fewer tokens, so it runs over what the first left in the shared
array), a one-token call, a matrix of per-block scales, and a request larger
than the array, which is refused before anything runs.
"""
import ctypes as C

import numpy as np
import pytest

from iris_amd import native, synth
from iris_amd.tensor import Q8Matrix
from oracle import cpu

pytestmark = pytest.mark.gpu

NOALLOC_BYTES = 32 << 20
E_SCRATCH = -6


@pytest.fixture(scope="module", autouse=True)
def device():
    native.check(native.lib().q8gpu_init(), "q8gpu_init")


def product_ws(m, x):
    L = native.lib()
    tokens = x.shape[0]
    dx = native.DeviceBuffer.from_array(x)
    dout = native.DeviceBuffer(tokens * m.rows * 4)
    ws_bytes = L.q8gpu_workspace_bytes(m.handle, tokens)
    ws = native.DeviceBuffer(max(ws_bytes, 1))
    native.check(L.q8gpu_product_device_ws(m.handle, dx.ptr, tokens, dout.ptr, ws.ptr, ws_bytes, None), "ws product")
    native.check(L.q8gpu_synchronize(), "synchronize")
    return dout.to_array(np.int32, (tokens, m.rows))


def product_noalloc(m, x):
    L = native.lib()
    tokens = x.shape[0]
    dx = native.DeviceBuffer.from_array(x)
    dout = native.DeviceBuffer(tokens * m.rows * 4)
    native.check(L.q8gpu_product_device_noalloc(m.handle, dx.ptr, tokens, dout.ptr, None), "noalloc product")
    native.check(L.q8gpu_synchronize(), "synchronize")
    return dout.to_array(np.int32, (tokens, m.rows))


def activations(rng, tokens, cols, bits):
    half = 1 << (bits - 1)
    return rng.integers(-half, half, (tokens, cols)).astype(np.int32)


def test_two_calls_in_a_row_match_the_work_space_entry_point():
    rows, cols = 300, 1024
    raw = synth.q8_matrix(synth.tensor_seed(41, 1), rows, cols, synth.scale_base_for(cols), True)
    m = Q8Matrix.from_bytes(raw, rows, cols)
    assert m.info()["scale_mode"] == "row"
    rng = np.random.default_rng(41)
    # First call: 96 tokens, some needing four digits; second: 40 tokens of
    # smaller values, run over the first call's planes and digit counts.
    first = activations(rng, 96, cols, 27)
    second = activations(rng, 40, cols, 12)
    for x in (first, second):
        print(f"noalloc product: {rows}x{cols}, {x.shape[0]} tokens", flush=True)
        got = product_noalloc(m, x)
        assert np.array_equal(got, product_ws(m, x))
        sample = x[:: max(1, x.shape[0] // 4)]
        want = cpu.linear_q8(sample, raw)
        assert np.array_equal(got[:: max(1, x.shape[0] // 4)], want)
    m.free()


def test_one_token_and_per_block_scales():
    rows, cols = 70, 512
    raw = synth.q8_matrix(synth.tensor_seed(42, 2), rows, cols, synth.scale_base_for(cols), False)
    m = Q8Matrix.from_bytes(raw, rows, cols)
    rng = np.random.default_rng(42)
    for tokens in (1, 33, 5):
        print(f"noalloc product: per-block scales, {tokens} tokens", flush=True)
        x = activations(rng, tokens, cols, 20)
        got = product_noalloc(m, x)
        assert np.array_equal(got, product_ws(m, x))
        assert np.array_equal(got, cpu.linear_q8(x, raw))
    # folded for the matrix cores: the same values through both entry points
    m.prepare_matrix_cores()
    for tokens in (33, 5):
        print(f"noalloc product: folded per-block scales, {tokens} tokens", flush=True)
        x = activations(rng, tokens, cols, 20)
        got = product_noalloc(m, x)
        assert np.array_equal(got, product_ws(m, x))
        assert np.array_equal(got, cpu.linear_q8(x, raw))
    m.free()


def test_larger_than_the_scratch_is_refused():
    rows, cols = 32, 4096
    raw = synth.q8_matrix(synth.tensor_seed(43, 1), rows, cols, synth.scale_base_for(cols), True)
    m = Q8Matrix.from_bytes(raw, rows, cols)
    L = native.lib()
    tokens = 2048  # 5 planes x 2048 tokens x 4096 values = 40 MiB of planes
    assert L.q8gpu_workspace_bytes(m.handle, tokens) > NOALLOC_BYTES
    dx = native.DeviceBuffer(tokens * cols * 4)
    dout = native.DeviceBuffer(tokens * rows * 4)
    rc = L.q8gpu_product_device_noalloc(m.handle, dx.ptr, tokens, dout.ptr, None)
    assert rc == E_SCRATCH
    assert "scratch" in native.error_text(rc)
    m.free()
