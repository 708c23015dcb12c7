"""GPU parity of the multi-row attention on the int8 matrix cores.

The narrow softmax routines are checked against the oracle's general ones
over every logit difference that can give a non-zero exp term and over
weight quotients chosen to hit each rounding case; the kernel itself
through teacher-forced passes of models with head sizes 64 and 128 (rows
across several 64-key steps and partial 16-row tiles), a Gemma model with
sliding windows, and a layer whose values need a fourth digit (the
workgroups take the scalar one-row routine there).
"""
import hashlib

import numpy as np
import pytest

from iris_amd import native, synth
from iris_amd.direct import DeviceModel, Session
from oracle import cpu

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def device():
    native.check(native.lib().q8gpu_init(), "q8gpu_init")


def _numerics(diff, e, s, dot, scale):
    n = diff.size
    L = native.lib()
    bufs = [native.DeviceBuffer.from_array(np.ascontiguousarray(a)) for a in (diff, e, s, dot)]
    dexp, dw, dsc = native.DeviceBuffer(8 * n), native.DeviceBuffer(4 * n), native.DeviceBuffer(4 * n)
    native.check(L.iris_attention_numerics(*[b.ptr for b in bufs], scale, n, dexp.ptr, dw.ptr, dsc.ptr), "numerics")
    return dexp.to_array(np.uint64, (n,)), dw.to_array(np.int32, (n,)), dsc.to_array(np.int32, (n,))


def test_attention_numerics_against_oracle():
    O = cpu.lib()
    # Every logit difference below the -16 cut, and a few at and past it.
    diff = np.arange(0, (1 << 20) + 8, dtype=np.uint32)
    diff = np.concatenate([diff, np.array([1 << 24, 1 << 31, 2 ** 32 - 1], np.uint32)])
    # Raw weights: e in [0, 2^32] against sums in [2^32, 4096 * 2^32), and
    # sums k * 2^32 with e = k/2 + j*k (k even): quotients ending in exactly
    # one half, so the ties-to-even step of div_acc is taken both ways.
    rng = np.random.default_rng(3)
    n = diff.size
    sums = rng.integers(1 << 32, 4096 << 32, n, dtype=np.uint64)
    es = rng.integers(0, (1 << 32) + 1, n, dtype=np.uint64)
    k = 2 * rng.integers(1, 2048, n // 4, dtype=np.uint64)
    sums[: n // 4] = k << np.uint64(32)
    es[: n // 4] = np.minimum(k // np.uint64(2) + k * rng.integers(0, 1 << 20, n // 4, dtype=np.uint64),
                              np.uint64(1 << 32))
    es[:3] = [0, 1 << 32, 1 << 32]
    sums[:3] = [1 << 32, 1 << 32, (1 << 33) + 2]
    # Scores: wrapping sums q0*k0 + q1*k1 of full-range i32 pairs, through
    # the oracle's two-element scaled_score (head size 128's scale).
    qk = rng.integers(-2 ** 31, 2 ** 31, (n, 4), dtype=np.int64)
    dots = ((qk[:, 0] * qk[:, 1]).astype(np.uint64) + (qk[:, 2] * qk[:, 3]).astype(np.uint64)).view(np.int64)
    scale = O.dn_attention_scale_q32(128)
    got_e, got_w, got_s = _numerics(diff, es, sums, dots, scale)
    want_e = np.array([O.dn_softmax_exp_term(-(int(d) << 16)) for d in diff], np.int64).astype(np.uint64)
    assert np.array_equal(got_e, want_e)
    want_w = np.array([O.dn_requantize(O.dn_div_acc(int(e), int(s))) for e, s in zip(es, sums)], np.int32)
    assert np.array_equal(got_w, want_w)
    idx = np.arange(0, n, 7)
    q2 = np.ascontiguousarray(qk[:, [0, 2]].astype(np.int32))
    k2 = np.ascontiguousarray(qk[:, [1, 3]].astype(np.int32))
    want_s = np.array([O.dn_scaled_score(q2[i], k2[i], 2, scale) for i in idx], np.int32)
    assert np.array_equal(got_s[idx], want_s)


def _check_pass(m, rows, max_positions=None):
    ids = synth.token_ids(11, rows, m.vocab)
    dm = DeviceModel(m)
    s = Session(dm, max_positions or rows, rows)
    got, hashes = s.layer_pass(ids)
    r = cpu.OracleRun(m, max_positions or rows)
    _, layers = r.pass_rows(list(ids), 0, keep_layers=True)
    for layer in range(m.num_layers):
        assert np.array_equal(got[layer], layers[layer]), layer
        assert hashes[layer] == hashlib.sha256(layers[layer].astype("<i4").tobytes()).hexdigest()
    s.free()
    dm.free()


@pytest.mark.parametrize("head_dim,heads,kv_heads,rows", [
    (128, 8, 2, 150), (64, 16, 2, 77), (128, 4, 1, 17),
    (64, 4, 2, 70), (128, 8, 8, 40), (256, 8, 1, 1030), (256, 16, 2, 520), (256, 8, 1, 90)])
def test_prefill_attention_mistral(head_dim, heads, kv_heads, rows):
    # GQA groups of one, two, four and eight (a workgroup's four heads on one
    # to four KV heads), head sizes 64, 128 and 256 (four value passes, from
    # 128 workgroups on: 1030 and 520 rows; 90 rows take the one-row
    # routine), partial query tiles and key steps.
    m = synth.mistral_model(512, 2, heads, kv_heads, head_dim, 512, 512, seed=31 + head_dim + rows)
    _check_pass(m, rows, max_positions=rows + 40)


def test_prefill_attention_large_values_take_the_scalar_routine():
    # Layer 0's attention norm weights scaled by 512: its values need four
    # digits, so its workgroups use the one-row routine; layer 1 stays on the
    # matrix cores.
    m = synth.mistral_model(512, 2, 8, 2, 64, 512, 512, seed=77)
    key = synth.PREFIX + "layers.0.input_layernorm.weight"
    m.tensors[key] = (m.tensors[key].astype(np.int64) * 512).clip(-2 ** 31, 2 ** 31 - 1).astype(np.int32)
    _check_pass(m, 70)


def test_prefill_attention_gemma_sliding_window():
    # Four query heads on one KV head; sliding layers of head size 64 with a
    # 40-key window (the first visible key moves inside the 64-key steps)
    # alternating with full layers of head size 128 and half rotary, the last
    # two layers reading earlier layers' caches.
    shape = synth.gemma_shape(256, 4, 4, 1, 64, 1024, 64, global_head_dim=128, sliding_window=40,
                              layer_types=["sliding_attention", "full_attention"] * 2, num_kv_shared_layers=2,
                              partial_rotary=0.5, softcap=30.0)
    m = synth.gemma_model(shape, 512, seed=5)
    _check_pass(m, 100)
    _check_pass(synth.tiny_gemma(), 33)


def test_silu_against_oracle():
    # The SwiGLU gate as the product epilogues compute it (narrow Horner
    # steps, the 2^63 quotient from a corrected double estimate): every value
    # in [-2^20, 2^20] in steps of 3, the ends of the range and random values.
    O = cpu.lib()
    rng = np.random.default_rng(9)
    x = np.concatenate([np.arange(-(1 << 20), (1 << 20) + 1, 3, dtype=np.int64),
                        np.array([0, 1, -1, 2 ** 31 - 1, -2 ** 31, 2 ** 31 - 2, -2 ** 31 + 1]),
                        rng.integers(-2 ** 31, 2 ** 31, 300000)]).astype(np.int32)
    dx = native.DeviceBuffer.from_array(x)
    dout = native.DeviceBuffer(4 * x.size)
    native.check(native.lib().iris_silu_device(dx.ptr, x.size, dout.ptr), "silu")
    got = dout.to_array(np.int32, (x.size,))
    want = np.array([O.dn_silu(int(v)) for v in x], np.int32)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("family", ["mistral", "gemma"])
def test_long_context_decode_matches_oracle(family):
    # One-row decode attention past several rounds of its key loop (512
    # positions per round at head size 128, 1024 at 64), with a sliding
    # window whose first visible position moves through every offset in a
    # group of four; every logit compared with the oracle.
    prompt_len, tokens, max_pos = 1030, 6, 1100
    if family == "mistral":
        m = synth.mistral_model(256, 2, 8, 2, 128, 512, 512, seed=41)
    else:
        shape = synth.gemma_shape(256, 2, 4, 1, 64, 512, 64, sliding_window=701,
                                  layer_types=["sliding_attention", "full_attention"])
        m = synth.gemma_model(shape, 512, seed=43)
    prompt = synth.token_ids(13, prompt_len, m.vocab)
    print(f"long-context decode, {family}", flush=True)
    dm = DeviceModel(m)
    s = Session(dm, max_pos, prompt_len)
    got = s.generate(prompt, tokens, keep_logits=True)
    r = cpu.OracleRun(m, max_pos)
    want_tokens, want_logits = r.generate(list(prompt), tokens, keep_logits=True)
    assert got.token_ids == want_tokens
    assert np.array_equal(got.logits, np.stack(want_logits))
    s.free()
    dm.free()


@pytest.mark.timeout(600)
def test_silu_every_input():
    # All 2^32 Q16.16 inputs, in chunks of 2^25: the device silu (the SwiGLU
    # gate of the product epilogues) and the table lookup of the matrix-core
    # epilogues (the table inside |x| < 1453635, x or 0 outside) against the
    # oracle's silu (mistral.rs:59-77).
    chunk = 1 << 25
    dx = native.DeviceBuffer(4 * chunk)
    dout = native.DeviceBuffer(4 * chunk)
    bad = bad_table = 0
    for c in range((1 << 32) // chunk):
        x = (np.arange(chunk, dtype=np.int64) + (c * chunk - (1 << 31))).astype(np.int32)
        native.check(native.lib().iris_memcpy_h2d(dx.ptr, x.ctypes.data, x.nbytes), "copy")
        native.check(native.lib().iris_silu_device(dx.ptr, chunk, dout.ptr), "silu")
        got = dout.to_array(np.int32, (chunk,))
        native.check(native.lib().iris_silu_table_device(dx.ptr, chunk, dout.ptr), "silu table")
        got_table = dout.to_array(np.int32, (chunk,))
        want = cpu.silu_many(x)
        bad += int(np.count_nonzero(got != want))
        bad_table += int(np.count_nonzero(got_table != want))
        if c % 32 == 31:
            print(f"silu: {(c + 1) * chunk} inputs checked, {bad} differ, {bad_table} by table", flush=True)
    assert bad == 0 and bad_table == 0
