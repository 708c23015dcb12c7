"""The reference's direct-executor fixtures on the GPU, through the C ABI:
a gemma-dense model of no layers loaded from a verified bundle, run by the
device token loop, against the loop outputs the reference's own tests expect
(crates/inference/direct/tests/executor.rs:141-189, 372-560)."""
import hashlib

import numpy as np
import pytest

from iris_amd import native
from iris_amd import artifacts
from iris_amd.direct import DeviceModel, Session
from oracle import cpu
from tests import executor_fixtures as fx

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def device():
    native.check(native.lib().q8gpu_init(), "q8gpu_init")


def _session(path):
    dm = DeviceModel.from_manifest(path)
    return dm, Session(dm, 16, 8)


@pytest.mark.parametrize("use_graph", [True, False])
def test_tiny_model_selects_token_2(tmp_path, use_graph):
    # :372-470: prompt "h" = [1], one token -> [2], hash of the JSON "[2]".
    print(f"zero-layer fixture, graph={use_graph}", flush=True)
    dm, s = _session(fx.write_tiny_bundle(str(tmp_path)))
    got = s.generate([1], 1, use_graph=use_graph)
    assert got.token_ids == [2]
    assert got.token_ids_sha256 == hashlib.sha256(b"[2]").hexdigest()
    assert got.stop_reason == "max_new_tokens"


@pytest.mark.parametrize("use_graph", [True, False])
@pytest.mark.parametrize("eos, expected", [(2, [2]), (0, [2, 0])])
def test_tiny_model_stops_at_eos(tmp_path, eos, expected, use_graph):
    # :479-531: budget 8, EOS {2} -> [2], EOS {0} -> [2, 0]; stop reason "eos".
    print(f"zero-layer fixture, eos={eos}, graph={use_graph}", flush=True)
    dm, s = _session(fx.write_tiny_bundle(str(tmp_path), eos_token_ids=[eos]))
    got = s.generate([1], 8, use_graph=use_graph)
    assert got.token_ids == expected
    assert got.stop_reason == "eos"
    assert got.token_ids_sha256 == hashlib.sha256(
        ("[" + ",".join(map(str, expected)) + "]").encode()).hexdigest()


def test_tiny_model_keeps_the_budget(tmp_path):
    # :533-560: prompt "hhhh" = [1, 1, 1, 1], budget 3 -> three tokens.
    print("zero-layer fixture, budget 3", flush=True)
    dm, s = _session(fx.write_tiny_bundle(str(tmp_path)))
    got = s.generate([1, 1, 1, 1], 3)
    assert len(got.token_ids) == 3 and got.token_ids[:2] == [2, 0]
    assert got.stop_reason == "max_new_tokens"


def test_head_tie_selects_the_earliest_id(tmp_path):
    # :141-189: row e0 against head rows {e0, 0, e0} -> token 0 from three
    # logits, the first and last equal.
    print("zero-layer fixture, head tie", flush=True)
    dm, s = _session(fx.write_head_tie_bundle(str(tmp_path)))
    got = s.generate([1], 1, keep_logits=True)
    assert got.token_ids == [0]
    lg = got.logits[0]
    assert lg.shape == (3,) and lg[0] == lg[2] > 0 and lg[1] == 0
    _, model, mapped = artifacts.load_model(dm.manifest.path)
    _, want = cpu.OracleRun(model, 16).generate([1], 1, keep_logits=True)
    mapped.close()
    assert np.array_equal(lg, want[0])


def _identity_layer_model():
    """The layer fixture of native_decode_rotary_outputs_match_prefill_across_chunks
    (crates/inference/direct/tests/executor.rs:190-350) as a one-layer
    gemma-dense model: every product the identity, norms ONE, q/k norms e0,
    RoPE base 10000 on the first pair only (partial rotary 2/32; pair 0's
    frequency is 1.0 whatever the frequency base), and PLE inputs of ONE
    (a zero model projection, PLE embedding rows of ONE, scales ONE). Token
    t embeds to ONE in every lane but lane 1, which is ONE for even t and
    -ONE for odd t (executor.rs:262-276)."""
    from iris_amd import model as model_mod
    from iris_amd.model import PREFIX
    W, ONE = fx.W, fx.ONE
    ident = fx.q8_exact(fx.one_hot_rows(range(W)))
    q8 = lambda vals: np.frombuffer(fx.q8_exact(vals), dtype=np.uint8).reshape(-1, 34).copy()
    rows = []
    for t in range(5):
        r = [ONE] * W
        r[1] = ONE if t % 2 == 0 else -ONE
        rows += r
    t = {PREFIX + "embed_tokens.weight": q8(rows),
         PREFIX + "embed_tokens_per_layer.weight": q8([ONE] * (5 * W)),
         PREFIX + "per_layer_model_projection.weight": np.zeros((W, W), dtype=np.int32),
         PREFIX + "per_layer_projection_norm.weight": np.full(W, ONE, dtype=np.int32),
         PREFIX + "norm.weight": np.full(W, ONE, dtype=np.int32)}
    at = PREFIX + "layers.0."
    for n in ("self_attn.q_proj.weight", "self_attn.k_proj.weight", "self_attn.v_proj.weight",
              "self_attn.o_proj.weight", "mlp.gate_proj.weight", "mlp.up_proj.weight", "mlp.down_proj.weight"):
        t[at + n] = np.frombuffer(ident, dtype=np.uint8).reshape(W, 34).copy()
    for n in ("per_layer_input_gate.weight", "per_layer_projection.weight"):
        t[at + n] = np.asarray(fx.one_hot_rows(range(W)), dtype=np.int32).reshape(W, W)
    for n in ("input_layernorm.weight", "post_attention_layernorm.weight", "pre_feedforward_layernorm.weight",
              "post_feedforward_layernorm.weight", "post_per_layer_input_norm.weight"):
        t[at + n] = np.full(W, ONE, dtype=np.int32)
    t[at + "self_attn.q_norm.weight"] = np.asarray(fx.one_hot_rows([0]), dtype=np.int32)
    t[at + "self_attn.k_norm.weight"] = np.asarray(fx.one_hot_rows([0]), dtype=np.int32)
    shape = model_mod.GemmaShape(
        hidden_size=W, num_hidden_layers=1, num_attention_heads=1, num_key_value_heads=1, head_dim=W,
        global_head_dim=W, vocab_size=5, hidden_size_per_layer_input=W, sliding_window=0,
        layer_types=["full_attention"], num_kv_shared_layers=0, norm_eps=0, rope_base_sliding=10_000 << 32,
        rope_base_full=10_000 << 32, full_partial_rotary_factor_q16=ONE * 2 // W, embedding_scale=ONE,
        ple_embedding_scale=ONE, ple_projection_scalar=ONE, ple_input_scale=ONE, final_logit_softcap=0,
        tied_head=True)
    return model_mod.Model("gemma-dense", shape, t)


def test_identity_layer_known_answer():
    # executor.rs:316-319: position 1's cached key starts [35408, 55146]; the
    # five rows as one pass and as the chunks (0,1), (1,2), (2,3), (3,5)
    # give the same rows and keys (:322-346), all equal to the oracle's.
    print("identity gemma layer known answer", flush=True)
    m = _identity_layer_model()
    assert m.rope_at(0)[1] == 2
    dm = DeviceModel(m)
    s = Session(dm, 8, 8)
    ids = [0, 1, 2, 3, 4]
    rows, hashes = s.layer_pass(ids)
    k, v = s.read_kv(0, 0, 5)
    assert list(k[1][:2]) == [35408, 55146]
    r = cpu.OracleRun(m, 8)
    _, layers = r.pass_rows(ids, 0, keep_layers=True)
    assert np.array_equal(rows[0], layers[0])
    assert np.array_equal(k, r.k_cache[0][:5]) and np.array_equal(v, r.v_cache[0][:5])
    s2 = Session(dm, 8, 8)
    for a, b in [(0, 1), (1, 2), (2, 3), (3, 5)]:
        got, _ = s2.layer_range(ids[a:b], a)
        assert np.array_equal(got[0], rows[0][a:b]), (a, b)
    k2, v2 = s2.read_kv(0, 0, 5)
    assert np.array_equal(k2, k) and np.array_equal(v2, v)
    s2.free()
    s.free()
    dm.free()
