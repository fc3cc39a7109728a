"""The oracle's layer compositions against golden vectors written by HF transformers' own Qwen3_5 modules
(tests/golden/make_layer_golden.py), plus invariants of the stack. CPU only."""
import os
import sys

import pytest
import torch
from safetensors.torch import load_file

import oracle
from oracle import model as om

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
from tiny_weights import STEER_LAYER, tiny_config, tiny_inputs, tiny_weights  # noqa: E402

GOLD = load_file(os.path.join(HERE, "golden", "qwen35_tiny_golden.safetensors"))
TOL = 2e-4


@pytest.fixture(scope="module")
def tiny():
    cfg = tiny_config()
    return cfg, tiny_weights(cfg)


def test_residual_stream_after_every_layer(tiny):
    cfg, W = tiny
    ids = GOLD["ids"]
    for l in range(cfg.layers):
        m = om.OracleModel(cfg, W, steer_layer=STEER_LAYER)
        _, resid = m.forward(ids, collect_layer=l, stop_after=l)
        e = oracle.rel_err(resid[:, ::7], GOLD[f"resid_l{l}"])
        assert e <= TOL, (l, e)


def test_prefill_and_cached_decode_logits(tiny):
    cfg, W = tiny
    m = om.OracleModel(cfg, W, steer_layer=STEER_LAYER)
    logits, _ = m.forward(GOLD["ids"])
    assert oracle.rel_err(logits, GOLD["logits_prefill"]) <= TOL
    assert torch.equal(logits.argmax(-1, keepdim=True), GOLD["next_ids"])
    logits2, _ = m.forward(GOLD["next_ids"])
    assert oracle.rel_err(logits2, GOLD["logits_decode"]) <= TOL


def test_residual_vector_after_layer(tiny):
    cfg, W = tiny
    _, vec = tiny_inputs(cfg)
    m = om.OracleModel(cfg, W, steer_layer=STEER_LAYER)
    m.set_vectors(torch.stack([vec, -vec]))
    logits, _ = m.forward(GOLD["ids"])
    assert oracle.rel_err(logits, GOLD["logits_steered"]) <= TOL


def test_decode_continues_prefill_and_rows_are_independent(tiny):
    """Prefill T then one decode step equals a fresh prefill of T + 1 (chunked vs recurrent delta rule, KV cache);
    a two-row batch equals each row alone."""
    cfg, W = tiny
    ids = GOLD["ids"]
    full = torch.cat([ids, GOLD["next_ids"]], dim=1)
    m = om.OracleModel(cfg, W)
    ref, _ = m.forward(full)
    m2 = om.OracleModel(cfg, W)
    m2.forward(ids)
    step, _ = m2.forward(GOLD["next_ids"])
    assert oracle.rel_err(step, ref) <= 1e-5
    m3 = om.OracleModel(cfg, W)
    row1, _ = m3.forward(ids[1:])
    m4 = om.OracleModel(cfg, W)
    both, _ = m4.forward(ids)
    assert oracle.rel_err(row1[0], both[1]) <= 1e-5


def test_median_residual_norm_convention():
    """Median over tokens 1..T-1 of the row norms, element len >> 1 of the sorted list (engine/analysis.js:64-74)."""
    x = torch.zeros(6, 3)
    x[:, 0] = torch.tensor([100.0, 1.0, 5.0, 3.0, 4.0, 2.0])  # token 0 is skipped
    assert om.median_resid_norm(x) == 3.0
