"""The oracle's token loop against the only end-to-end loop outputs the
reference holds: its direct-executor fixtures
(crates/inference/direct/tests/executor.rs:141-189, 372-560), loaded from a
verified bundle as the executor loads them."""
import numpy as np
import pytest

from iris_amd import artifacts
from oracle import cpu
from tests import executor_fixtures as fx


def _oracle(path):
    _, model, mapped = artifacts.load_model(path)
    return cpu.OracleRun(model, 16), model, mapped


def test_tiny_model_selects_token_2(tmp_path):
    # direct_executor_runs_from_direct_manifest_without_raster_toml (:372-470):
    # prompt "h" = [1], one token -> [2].
    run, model, mapped = _oracle(fx.write_tiny_bundle(str(tmp_path)))
    tokens, _ = run.generate([1], 1)
    assert tokens == [2]
    mapped.close()


@pytest.mark.parametrize("eos, expected", [(2, [2]), (0, [2, 0])])
def test_tiny_model_stops_at_eos(tmp_path, eos, expected):
    # direct_executor_stops_at_eos_and_reports_only_selected_tokens (:479-531):
    # budget 8; the model selects 2, then 0 after embedding 2.
    run, model, mapped = _oracle(fx.write_tiny_bundle(str(tmp_path), eos_token_ids=[eos]))
    tokens, _ = run.generate([1], 8)
    assert tokens == expected
    mapped.close()


def test_tiny_model_keeps_the_budget(tmp_path):
    # direct_executor_keeps_a_maximum_budget_when_no_eos_is_selected (:533-560):
    # prompt "hhhh" = [1, 1, 1, 1], budget 3 -> three tokens.
    run, model, mapped = _oracle(fx.write_tiny_bundle(str(tmp_path)))
    tokens, _ = run.generate([1, 1, 1, 1], 3)
    assert len(tokens) == 3 and tokens[:2] == [2, 0]
    mapped.close()


def test_head_tie_selects_the_earliest_id(tmp_path):
    # final_head_logits_feed_shared_decode_select_tie_break (:141-189):
    # row e0 against head rows {e0, 0, e0} -> three logits, token 0.
    run, model, mapped = _oracle(fx.write_head_tie_bundle(str(tmp_path)))
    tokens, logits = run.generate([1], 1, keep_logits=True)
    assert tokens == [0]
    lg = logits[0]
    assert lg.shape == (3,) and lg[0] == lg[2] > 0 and lg[1] == 0
    mapped.close()


def test_q8_exact_blocks():
    # ONE alone: k = 0, scale 1.0 (f16 0x3c00), weight 1; ONE/2 needs k = 1.
    b = fx.q8_exact(fx.one_hot_rows([0]))
    assert b[:2] == bytes([0x00, 0x3C]) and b[2] == 1 and not any(b[3:])
    half = fx.q8_exact([fx.ONE // 2] + [0] * 31)
    assert half[:2] == bytes([0x00, 0x38]) and half[2] == 1
    with pytest.raises(ValueError):
        fx.q8_exact([1] * 31 + [fx.ONE * 200])


def test_gemma_layer_known_answer_through_the_whole_layer():
    # native_decode_rotary_outputs_match_prefill_across_chunks
    # (crates/inference/direct/tests/executor.rs:190-350): one gemma-dense
    # layer, 32 wide, every product the identity (exact Q8_0, and Q16.16 for
    # the PLE matrices), norms ONE, q/k norms the one-hot e0, RoPE base
    # 10000 on the first pair (rotary 2, frequency base 2), over five rows
    # of ONE with lane 1 at +-ONE: position 1's cached key starts
    # [35408, 55146] (:316-319). This pins the layer's key path end to end:
    # input norm, product, k norm, rotation, cache store. The same layer
    # over the chunks (0,1), (1,2), (2,3), (3,5) reproduces the one pass's
    # rows and keys (:322-346).
    import ctypes as C
    W = fx.W
    ONE = fx.ONE
    identity = fx.one_hot_rows(range(W))
    q8_id = np.frombuffer(fx.q8_exact(identity), dtype=np.uint8).reshape(W, 34)
    i32_id = np.asarray(identity, dtype=np.int32).reshape(W, W)
    keep = []

    def hold(a, dtype):
        a = np.ascontiguousarray(a, dtype=dtype)
        keep.append(a)
        return a.ctypes.data

    L = cpu.GemmaLayerC()
    L.hidden = L.ffn = W
    L.heads = L.kv_heads = 1
    L.head_dim = W
    L.ple_width = W
    L.sliding_window = 0
    L.layer_scalar = 0
    L.norm_eps = 0
    L.rope_base = 10_000 << 32
    L.rotary_dim = 2
    L.rope_freq_base_dim = 2
    norm = [ONE] * W
    unit = fx.one_hot_rows([0])
    for f in ("norm_input", "norm_post_attn", "norm_pre_ffw", "norm_post_ffw", "ple_post_norm"):
        setattr(L, f, hold(norm, np.int32))
    L.q_norm = hold(unit, np.int32)
    L.k_norm = hold(unit, np.int32)
    for f in ("w_q", "w_k", "w_v", "w_o", "w_gate", "w_up", "w_down"):
        setattr(L, f, hold(q8_id, np.uint8))
    L.ple_input_gate = hold(i32_id, np.int32)
    L.ple_layer_projection = hold(i32_id, np.int32)

    rows = np.full((5, W), ONE, dtype=np.int32)
    rows[1::2, 1] = -ONE
    ple = np.full((5, W), ONE, dtype=np.int32)

    def run(x, start, k, v):
        out = np.empty_like(x)
        rc = cpu.lib().orc_gemma_layer_forward(C.byref(L), np.ascontiguousarray(x), x.shape[0], start, k, v, k, v,
                                              np.ascontiguousarray(ple[start:start + x.shape[0]]), out, 1)
        assert rc == 0
        return out

    k_all = np.zeros((8, W), dtype=np.int32)
    v_all = np.zeros((8, W), dtype=np.int32)
    whole = run(rows, 0, k_all, v_all)
    assert list(k_all[1][:2]) == [35408, 55146]
    k = np.zeros((8, W), dtype=np.int32)
    v = np.zeros((8, W), dtype=np.int32)
    for a, b in [(0, 1), (1, 2), (2, 3), (3, 5)]:
        got = run(rows[a:b], a, k, v)
        assert np.array_equal(got, whole[a:b]), (a, b)
        assert np.array_equal(k[:b], k_all[:b]) and np.array_equal(v[:b], v_all[:b]), (a, b)
