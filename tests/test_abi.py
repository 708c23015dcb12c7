"""The C ABI library loads and exports every function include/iris_hip.h
declares (no device calls: this runs without a GPU)."""
import ctypes as C
import os

import pytest

from iris_amd import native


def test_library_is_built():
    assert os.path.exists(native.LIB_PATH), "run `python -m iris_amd.build` first"


def test_every_declared_function_is_exported():
    names = native.header_functions()
    assert "q8gpu_product" in names and "q8gpu_upload" in names
    lib = C.CDLL(native.LIB_PATH)
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_reference_drop_in_symbols_are_present():
    # The five symbols crates/inference/kernels/src/gpu.rs:45-62 links against.
    lib = C.CDLL(native.LIB_PATH)
    for n in ["q8gpu_error", "q8gpu_init", "q8gpu_upload", "q8gpu_free", "q8gpu_product"]:
        assert hasattr(lib, n)


def test_error_text_without_a_device():
    assert native.error_text(-2) == "Q8_0 block scale is not finite"
    assert native.error_text(-1)


def test_layer_hash_is_sha256():
    # FIPS 180-4 vectors plus lengths around the padding boundary.
    import hashlib
    from iris_amd.direct import sha256
    import numpy as np
    rng = np.random.default_rng(5)
    longer = [rng.integers(0, 256, n, dtype=np.uint8).tobytes() for n in (1000, 65536 + 17, 3 << 20)]
    for data in [b"", b"abc", b"a" * 55, b"a" * 56, b"a" * 64, bytes(range(256)) * 9] + longer:
        assert sha256(data) == hashlib.sha256(data).hexdigest()
    assert sha256(b"abc") == "ba7816bf8f01cfea414140de5dae2223b00361a396177a9cb410ff61f20015ad"


def test_no_kernel_tracer_in_the_test_process():
    # Graph replays are refused only under a kernel tracer; the tests run
    # without one, so the graph cases run rather than being refused.
    assert native.kernel_tracer_loaded() is False
    assert "kernel tracer" in native.error_text(-7)
