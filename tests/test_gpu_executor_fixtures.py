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
