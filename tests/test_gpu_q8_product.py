"""GPU parity of the Q8_0 product against the oracle, through the C ABI.

Cases follow the reference's own device tests
(crates/inference/kernels/src/gpu.rs:374-495): shapes on and across tiles,
three magnitude regimes including i32::MIN/MAX activations, exact ties, a
matrix uploaded through both entry points, and non-finite scales refused.
Plus the microbenchmark's full sizes (the M=1 GEMV at K=4096, N=14336 and
the M=512 GEMM at K=N=4096).
"""
import numpy as np
import pytest

from iris_amd import native, synth
from iris_amd.tensor import Q8Matrix, linear_slab_from_source
from oracle import cpu

pytestmark = pytest.mark.gpu


def rand_matrix(rng, rows, cols, max_exponent):
    """Every weight byte, finite scales of either sign up to max_exponent (gpu.rs:322-334)."""
    nb = rows * cols // 32
    v = rng.integers(0, 1 << 62, nb, dtype=np.int64)
    exponent = (v >> 20) % (max_exponent + 1)
    bits = ((v & 1) << 15) | (exponent << 10) | ((v >> 4) & 0x3FF)
    raw = np.empty((nb, 34), np.uint8)
    raw[:, 0], raw[:, 1] = bits & 0xFF, (bits >> 8) & 0xFF
    raw[:, 2:] = rng.integers(0, 256, (nb, 32))
    return raw.reshape(rows, -1)


def rand_activations(rng, tokens, cols, magnitude_bits):
    """i32::MAX / i32::MIN / 0 at 1/61 of positions, else magnitude_bits wide (gpu.rs:336-351)."""
    r = rng.integers(0, 1 << 62, (tokens, cols), dtype=np.int64)
    vals = ((r >> 16) & 0xFFFFFFFF).astype(np.uint32).view(np.int32) >> (32 - magnitude_bits)
    sel = r % 61
    vals = np.where(sel == 0, np.int32(2 ** 31 - 1), np.where(sel == 1, np.int32(-2 ** 31), np.where(sel == 2, 0, vals)))
    return vals.astype(np.int32)


@pytest.fixture(scope="module", autouse=True)
def device():
    native.check(native.lib().q8gpu_init(), "q8gpu_init")


# (200, 4160, 1) and (64, 8224, 1): one-row products whose waves stage their
# own blocks' planes (8- and 16-wave workgroups, a block count that leaves
# the last run of four blocks partial).
@pytest.mark.parametrize("rows,cols,tokens", [(1, 32, 1), (16, 32, 16), (17, 64, 15), (130, 96, 33), (300, 1536, 70),
                                              (200, 4160, 1), (64, 8224, 1), (48, 4096, 2)])
@pytest.mark.parametrize("max_exponent,magnitude_bits", [(30, 32), (18, 20), (5, 12)])
def test_products_equal_one_dot_row_per_value(rows, cols, tokens, max_exponent, magnitude_bits):
    print(f"shape {rows}x{cols} tokens {tokens} regime {max_exponent}/{magnitude_bits}", flush=True)
    rng = np.random.default_rng(rows * 7919 + cols * 31 + tokens + max_exponent)
    raw = rand_matrix(rng, rows, cols, max_exponent)
    x = rand_activations(rng, tokens, cols, magnitude_bits)
    m = Q8Matrix.from_bytes(raw, rows, cols)
    got = linear_slab_from_source(x, m)
    want = cpu.linear_q8(x, raw)
    assert np.array_equal(got, want)


def test_products_round_ties_to_even():
    # gpu.rs:397-418: scale 2^-15, activations in steps of 2^-2.
    rows, cols, tokens = 64, 32, 96
    raw = np.zeros((rows, 34), np.uint8)
    raw[:, 0], raw[:, 1] = 0x00, 0x02
    for row in range(rows):
        raw[row, 2 + row % 32] = np.uint8(np.int8([1, -1, 3, -3, 5, -7, 127, -128][row % 8]))
    idx = np.arange(tokens * cols)
    x = (((idx // cols) - 48 + (idx % cols)) << 14).astype(np.int32).reshape(tokens, cols)
    got = linear_slab_from_source(x, Q8Matrix.from_bytes(raw, rows, cols))
    assert np.array_equal(got, cpu.linear_q8(x, raw))


def test_reference_upload_entry_point_and_wide_scales():
    rng = np.random.default_rng(11)
    rows, cols, tokens = 130, 96, 33
    raw = rand_matrix(rng, rows, cols, 18)
    x = rand_activations(rng, tokens, cols, 20)
    blocks = raw.reshape(-1, 34)
    weights = blocks[:, 2:].view(np.int8).reshape(rows, cols)
    bits = blocks[:, 0].astype(np.int64) | (blocks[:, 1].astype(np.int64) << 8)
    e, mant = (bits >> 10) & 31, bits & 1023
    q24 = np.where(e == 0, mant, (1024 + mant) << np.maximum(e - 1, 0))
    q24 = np.where(bits & 0x8000, -q24, q24).reshape(rows, cols // 32)
    via_f16 = Q8Matrix.from_weights_and_scales(weights, q24)
    assert via_f16.info()["scale_mode"] == "f16"
    assert np.array_equal(linear_slab_from_source(x, via_f16), cpu.linear_q8(x, raw))
    # Scales no f16 can hold stay i64 per block; the product is still exact.
    wide = q24 * 3 + 1
    m = Q8Matrix.from_weights_and_scales(weights, wide)
    assert m.info()["scale_mode"] == "i64"
    got = linear_slab_from_source(x, m)
    for t in range(0, tokens, 5):
        for r in range(0, rows, 7):
            total = sum(int(np.dot(weights[r, b * 32:(b + 1) * 32].astype(np.int64),
                                   x[t, b * 32:(b + 1) * 32].astype(np.int64))) * int(wide[r, b])
                        for b in range(cols // 32))
            fl, rem = total >> 24, total & ((1 << 24) - 1)
            want = fl + 1 if rem > (1 << 23) or (rem == (1 << 23) and fl & 1) else fl
            assert got[t, r] == max(-2 ** 31, min(2 ** 31 - 1, want))


def test_uniform_row_scales_take_the_row_path():
    m = synth.q8_matrix(123, 48, 256, 0x0C00, per_row_scale=True)
    q = Q8Matrix.from_bytes(m, 48, 256)
    assert q.info()["scale_mode"] == "row"
    rng = np.random.default_rng(4)
    x = rand_activations(rng, 9, 256, 32)
    assert np.array_equal(linear_slab_from_source(x, q), cpu.linear_q8(x, m))


def test_non_finite_scales_are_refused():
    raw = np.zeros((1, 34), np.uint8)
    raw[0, 1] = 0x7C
    with pytest.raises(native.IrisError) as e:
        Q8Matrix.from_bytes(raw, 1, 32)
    assert e.value.code == -2


def test_no_tokens_and_width_mismatch():
    m = Q8Matrix.from_bytes(np.zeros((4, 34), np.uint8), 4, 32)
    assert linear_slab_from_source(np.zeros((0, 32), np.int32), m).shape == (0, 4)
    with pytest.raises(ValueError):
        linear_slab_from_source(np.zeros((2, 64), np.int32), m)


@pytest.mark.parametrize("per_row_scale", [True, False])
def test_microbench_gemv_full_size(per_row_scale):
    # The microbenchmark GEMV: M=1, K=4096, N=14336, every output.
    N, K = 14336, 4096
    raw = synth.q8_matrix(synth.tensor_seed(2, 1), N, K, synth.scale_base_for(K), per_row_scale)
    rng = np.random.default_rng(2)
    s_t = 256 + int(rng.integers(0, 256))
    x = (rng.integers(-127, 128, (1, K)) * s_t).astype(np.int32)
    m = Q8Matrix.from_bytes(raw, N, K)
    assert m.info()["scale_mode"] == ("row" if per_row_scale else "f16")
    assert np.array_equal(linear_slab_from_source(x, m), cpu.linear_q8(x, raw))


def test_microbench_gemm_full_size_sampled_rows():
    # The microbenchmark GEMM: M=512, K=N=4096; every token of
    # 96 sampled rows against the oracle, plus the stress (full-range) set.
    N, K, M = 4096, 4096, 512
    raw = synth.q8_matrix(synth.tensor_seed(2, 2), N, K, synth.scale_base_for(K), True)
    rng = np.random.default_rng(3)
    s = (256 + rng.integers(0, 256, (M, 1))).astype(np.int64)
    x = (rng.integers(-127, 128, (M, K)) * s).astype(np.int32)
    m = Q8Matrix.from_bytes(raw, N, K)
    got = linear_slab_from_source(x, m)
    rows = rng.choice(N, 96, replace=False)
    assert np.array_equal(got[:, rows], cpu.linear_q8(x, raw[rows]))
    xs = rand_activations(rng, 64, K, 32)
    got = linear_slab_from_source(xs, m)
    assert np.array_equal(got[:, rows], cpu.linear_q8(xs, raw[rows]))


@pytest.mark.parametrize("tokens,rows,cols", [(2, 16, 64), (65, 200, 128), (130, 300, 1536)])
def test_mfma_product_with_workspace(tokens, rows, cols):
    # Multi-token products of a row-scale matrix with caller work space run on
    # the int8 matrix cores; every output against the oracle, with partial
    # token and row tiles and full-range activations (five digit planes).
    rng = np.random.default_rng(tokens * 7 + rows)
    raw = synth.q8_matrix(synth.tensor_seed(9, rows), rows, cols, synth.scale_base_for(cols), True)
    m = Q8Matrix.from_bytes(raw, rows, cols)
    assert m.info()["scale_mode"] == "row"
    L = native.lib()
    for x in (rand_activations(rng, tokens, cols, 32), rand_activations(rng, tokens, cols, 20)):
        ws_bytes = L.q8gpu_workspace_bytes(m.handle, tokens)
        assert ws_bytes >= 5 * tokens * cols
        dx = native.DeviceBuffer.from_array(x)
        dout = native.DeviceBuffer(tokens * rows * 4)
        ws = native.DeviceBuffer(ws_bytes)
        assert L.q8gpu_product_device_ws(m.handle, dx.ptr, tokens, dout.ptr, ws.ptr, ws_bytes - 1, None) == -5
        native.check(L.q8gpu_product_device_ws(m.handle, dx.ptr, tokens, dout.ptr, ws.ptr, ws_bytes, None), "product")
        native.check(L.q8gpu_synchronize(), "sync")
        assert np.array_equal(dout.to_array(np.int32, (tokens, rows)), cpu.linear_q8(x, raw))


def product_ws(m, x):
    """q8gpu_product_device_ws with its work space: every output of x's tokens."""
    L = native.lib()
    tokens = x.shape[0]
    ws_bytes = L.q8gpu_workspace_bytes(m.handle, tokens)
    dx = native.DeviceBuffer.from_array(x)
    dout = native.DeviceBuffer(tokens * m.rows * 4)
    ws = native.DeviceBuffer(ws_bytes)
    native.check(L.q8gpu_product_device_ws(m.handle, dx.ptr, tokens, dout.ptr, ws.ptr, ws_bytes, None), "product")
    native.check(L.q8gpu_synchronize(), "sync")
    return dout.to_array(np.int32, (tokens, m.rows))


def grouped_activations(rng, tokens, cols):
    """Token group g (128 tokens each) needs exactly 1, 2, 3, 4, 5 digits for
    g = 0..4: magnitudes of 8, 15, 23 and 31 bits, then the full range with
    i32::MAX / i32::MIN at 1/61 of positions."""
    x = np.empty((tokens, cols), np.int32)
    for g0 in range(0, tokens, 128):
        g = (g0 // 128) % 5
        n = min(128, tokens - g0)
        if g < 4:
            b = (8, 15, 23, 31)[g]
            x[g0:g0 + n] = rng.integers(-(1 << (b - 1)), 1 << (b - 1), (n, cols))
        else:
            x[g0:g0 + n] = rand_activations(rng, n, cols, 32)
    return x


@pytest.mark.parametrize("tokens,rows,cols", [(603, 1024, 192), (603, 136, 4160), (300, 272, 64), (300, 22100, 128),
                                              (200, 32768, 64), (603, 1024, 256), (603, 136, 4224),
                                              (603, 136, 8192)])
def test_mfma_product_digit_paths(tokens, rows, cols):
    # Every digit count's code path (one to three planes side by side, four
    # and five in two token halves), one-step, short and long k loops,
    # launches whose block count does and does not split evenly over the
    # XCDs, and both workgroup shapes (256-row blocks when the launch fills
    # every CU: the fourth and fifth cases). The 128-row shapes split an
    # even number of 64-wide k steps between two wave groups (the last three
    # cases; rows of 8192 or more take the deeper rings, three stages at
    # three planes) and walk an odd number in one (the first three).
    rng = np.random.default_rng(tokens + rows + cols)
    raw = synth.q8_matrix(synth.tensor_seed(11, rows), rows, cols, synth.scale_base_for(cols), True)
    m = Q8Matrix.from_bytes(raw, rows, cols)
    L = native.lib()
    x = grouped_activations(rng, tokens, cols)
    ws_bytes = L.q8gpu_workspace_bytes(m.handle, tokens)
    dx = native.DeviceBuffer.from_array(x)
    dout = native.DeviceBuffer(tokens * rows * 4)
    ws = native.DeviceBuffer(ws_bytes)
    native.check(L.q8gpu_product_device_ws(m.handle, dx.ptr, tokens, dout.ptr, ws.ptr, ws_bytes, None), "product")
    native.check(L.q8gpu_synchronize(), "sync")
    assert np.array_equal(dout.to_array(np.int32, (tokens, rows)), cpu.linear_q8(x, raw))


def test_mfma_product_wide_row_scales():
    # Row-scale matrices whose Q.24 scales run from zero and subnormals up to
    # f16 exponent 30 (about 2^40), both signs, against full-range
    # activations with every magnitude from 8 to 32 bits: the MFMA epilogue's
    # 64-bit rounding path, its bit-length test near 2^63 and its 128-bit
    # redo all run; every output is compared.
    rng = np.random.default_rng(31)
    rows, cols, tokens = 512, 1024, 96
    nb = cols // 32
    exponent = np.concatenate([rng.integers(0, 12, 128), rng.integers(12, 22, 128), rng.integers(22, 31, 256)])
    bits = ((rng.integers(0, 2, rows) << 15) | (exponent << 10) | rng.integers(0, 1024, rows)).astype(np.int64)
    bits[:3] = [0, 0x8000, 0x0001]  # zero, negative zero, the smallest subnormal
    raw = np.empty((rows, nb, 34), np.uint8)
    raw[:, :, 0] = (bits & 0xFF)[:, None]
    raw[:, :, 1] = (bits >> 8)[:, None]
    raw[:, :, 2:] = rng.integers(0, 256, (rows, nb, 32))
    raw = raw.reshape(rows, -1)
    m = Q8Matrix.from_bytes(raw, rows, cols)
    assert m.info()["scale_mode"] == "row"
    x = np.concatenate([rand_activations(rng, 1, cols, int(b)) for b in np.linspace(8, 32, tokens).astype(int)])
    got = product_ws(m, x)
    assert np.array_equal(got, cpu.linear_q8(x, raw))


def per_block_matrix(rng, rows, cols, kind):
    """Q8_0 rows with one f16 scale per block, both signs, every weight
    byte: `kind` sets how the scales of a row spread (so how many digit
    planes the folded weights need): "tiny" subnormal scales below 2^-17
    (one or two planes), "same" one exponent per row with random
    significands (three), "unit" scales of 0 or 2^-24 (one plane, or two
    where a negative scale meets q = -128: w' = 128),
    "spread4" exponents within 4 binary orders
    (three), "spread12" within 12 (four), "wide" over 20 orders (five),
    "widest" every exponent 0..30 with subnormals beside the largest
    scales (six: the widest spread an f16 scale row can have), "top"
    exponents 26..30 (results saturate), plus zero scales and all-zero
    rows."""
    nb = cols // 32
    base = rng.integers(1, 17, (rows, 1))
    if kind == "widest":
        e = rng.integers(0, 31, (rows, nb))
        e[:, 0], e[:, -1] = 0, 30  # a subnormal block and an exponent-30 block in every row
        mant = rng.integers(1, 1024, (rows, nb))
    elif kind == "tiny":
        e = np.zeros((rows, nb), np.int64)
        mant = rng.integers(0, 96, (rows, nb))
    elif kind == "unit":
        e = np.zeros((rows, nb), np.int64)
        mant = rng.integers(0, 2, (rows, nb))
    else:
        spread = {"same": 0, "spread4": 4, "spread12": 12, "wide": 20, "top": 4}[kind]
        lo = rng.integers(26, 27, (rows, 1)) if kind == "top" else base
        e = lo + rng.integers(0, spread + 1, (rows, nb))
        mant = rng.integers(0, 1024, (rows, nb))
    bits = (rng.integers(0, 2, (rows, nb)) << 15) | (np.minimum(e, 30) << 10) | mant
    bits[rng.random((rows, nb)) < 0.02] = 0  # zero scales
    bits[::37] = 0                           # all-zero rows
    raw = np.empty((rows, nb, 34), np.uint8)
    raw[:, :, 0] = bits & 0xFF
    raw[:, :, 1] = bits >> 8
    raw[:, :, 2:] = rng.integers(0, 256, (rows, nb, 32))
    return raw.reshape(rows, -1)


@pytest.mark.parametrize("kind,planes", [("unit", None), ("tiny", None), ("same", 3), ("spread4", 3),
                                         ("spread12", 4), ("wide", 5), ("widest", 6), ("top", 3)])
@pytest.mark.parametrize("tokens,rows,cols", [(603, 200, 128), (129, 136, 4160)])
def test_per_block_scales_on_the_matrix_cores(kind, planes, tokens, rows, cols):
    # Per-block scale matrices folded into weight digit planes for the int8
    # matrix cores, one to six planes (every spread an f16 scale row can
    # have folds): every digit count of the activations (token groups of
    # 1..5 digits), partial row and token tiles, every output against the
    # oracle's dot_row. (None: the count depends on the draw.)
    rng = np.random.default_rng(tokens + rows + len(kind))
    raw = per_block_matrix(rng, rows, cols, kind)
    m = Q8Matrix.from_bytes(raw, rows, cols)
    assert m.info()["scale_mode"] == "f16"
    before = m.info()["bytes"]
    x = grouped_activations(rng, tokens, cols)
    want = cpu.linear_q8(x, raw)
    # Unprepared: the vector path, and the product allocates nothing.
    assert np.array_equal(product_ws(m, x), want)
    assert m.info()["bytes"] == before
    m.prepare_matrix_cores()
    # The folded planes were built: one byte per weight per plane (rows
    # padded to whole 16-row tiles), plus one 32-bit shift per row.
    tiles = (rows + 15) // 16
    extra = m.info()["bytes"] - before - tiles * 16 * 4
    assert extra > 0 and extra % (tiles * 16 * cols) == 0
    if planes is not None:
        assert extra // (tiles * 16 * cols) == planes
    got = product_ws(m, x)
    assert np.array_equal(got, want)
    # again, from the folded planes already there
    x2 = rand_activations(rng, 70, cols, 24)
    assert np.array_equal(product_ws(m, x2), cpu.linear_q8(x2, raw))
    # the no-allocation entry point gives the same values
    L = native.lib()
    dx = native.DeviceBuffer.from_array(x2)
    dout = native.DeviceBuffer(70 * rows * 4)
    native.check(L.q8gpu_product_device_noalloc(m.handle, dx.ptr, 70, dout.ptr, None), "noalloc")
    native.check(L.q8gpu_synchronize(), "sync")
    assert np.array_equal(dout.to_array(np.int32, (70, rows)), cpu.linear_q8(x2, raw))


def test_per_block_gemm_at_the_benchmark_shape_sampled():
    # The gate|up shape of the 2048-row pass with per-block scales (the
    # reference bundles' layout: base + next % 64 significands, generate.py:59):
    # sampled rows of every token against the oracle.
    rows, cols, tokens = 28672, 4096, 2048
    raw = synth.q8_matrix(synth.tensor_seed(12, 1), rows, cols, synth.scale_base_for(cols), False)
    m = Q8Matrix.from_bytes(raw, rows, cols)
    assert m.info()["scale_mode"] == "f16"
    m.prepare_matrix_cores()
    rng = np.random.default_rng(12)
    x = rng.integers(-(1 << 20), 1 << 20, (tokens, cols)).astype(np.int32)
    got = product_ws(m, x)
    sel = np.sort(rng.choice(rows, 96, replace=False))
    assert np.array_equal(got[:, sel], cpu.linear_q8(x, raw[sel]))
