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
