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
from tiny_weights import PUSH_LAYER, PUSH_NEURON, PUSH_VALUE, STEER_LAYER, tiny_config, tiny_inputs, \
    tiny_weights  # noqa: E402

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


def test_mlp_activation_capture_and_push_against_hf_hooks(tiny):
    """The oracle's captured MLP activations (the down_proj input) equal HF's forward pre-hook on down_proj
    (tests/engine_ref.py:11-20) for the prefill and the cached decode step, and with a neuron push on one layer the
    activations of every layer and the logits follow HF's pushed run."""
    cfg, W = tiny
    layers = tuple(range(cfg.layers))
    m = om.OracleModel(cfg, W)
    m.forward(GOLD["ids"], capture_layers=layers)
    for l in layers:
        assert oracle.rel_err(m.acts[l][:, ::7], GOLD[f"acts_l{l}"]) <= TOL, l
    m.forward(GOLD["next_ids"], capture_layers=layers)
    for l in layers:
        assert oracle.rel_err(m.acts[l][:, 0], GOLD[f"acts_decode_l{l}"]) <= TOL, l
    m = om.OracleModel(cfg, W)
    m.set_pushes({PUSH_LAYER: [(PUSH_NEURON, "add", [PUSH_VALUE] * 2)]})
    logits, _ = m.forward(GOLD["ids"], capture_layers=layers)
    for l in layers:
        assert oracle.rel_err(m.acts[l][:, ::7], GOLD[f"acts_push_l{l}"]) <= TOL, l
    assert oracle.rel_err(logits, GOLD["logits_pushed"]) <= TOL
    # the push must show: the unpushed run differs from the pushed fixture
    assert oracle.rel_err(GOLD["acts_l3"], GOLD["acts_push_l3"]) > 10 * TOL


def test_residual_snapshots_and_activations_compose(tiny):
    """The hook outputs fit the layer's algebra: resid after layer l = resid after its mixer + acts_l @ down_proj^T
    (+ the steering vector after the steer layer), and the last snapshot is the collected residual."""
    cfg, W = tiny
    ids, vec = tiny_inputs(cfg)
    m = om.OracleModel(cfg, W, steer_layer=STEER_LAYER)
    m.set_vectors(torch.stack([vec, -vec]))
    _, collected = m.forward(ids[:, :20], collect_layer=cfg.layers - 1, capture_layers=range(cfg.layers))
    assert len(m.resid_layer) == len(m.resid_mixer) == cfg.layers
    assert torch.equal(m.resid_layer[-1], collected)
    for l in range(cfg.layers):
        x = m.resid_mixer[l] + m.acts[l] @ om.dequant(W, f"layers.{l}.down_proj").T
        if l == STEER_LAYER:
            x = x + torch.stack([vec, -vec])[:, None, :]
        assert torch.allclose(x, m.resid_layer[l], rtol=0, atol=0), l


def test_head_scales_scale_each_heads_contribution(tiny):
    """Per-head output scales (engine/model.js:362-368) act linearly on the GDN mixer output: scales of 1 change
    nothing (bitwise), 0 on every head silences the mixer, the one-hot scales of the heads sum to the unscaled
    output, and mixed scales give the matching combination of the one-hot outputs."""
    cfg, W = tiny
    ids = GOLD["ids"][:, :24]
    B, T = ids.shape
    h = W["embed"][ids]

    def y_of(hs):
        y, _ = om.gdn_layer(cfg, W, 0, h, None, False, hs)
        return y
    y0 = y_of(None)
    assert torch.equal(y_of(torch.ones(cfg.lin_v_heads)), y0)
    assert torch.count_nonzero(y_of(torch.zeros(cfg.lin_v_heads))) == 0
    parts = sum(y_of(torch.eye(cfg.lin_v_heads)[i]) for i in range(cfg.lin_v_heads))
    assert oracle.rel_err(parts, y0) <= 1e-6
    y2 = y_of(torch.tensor([2.0, 0.5]))
    assert oracle.rel_err(y2, 2.0 * y_of(torch.tensor([1.0, 0.0])) + 0.5 * y_of(torch.tensor([0.0, 1.0]))) <= 1e-6


def test_median_residual_norm_convention():
    """Median over tokens 1..T-1 of the row norms, element len >> 1 of the sorted list (engine/analysis.js:64-74)."""
    x = torch.zeros(6, 3)
    x[:, 0] = torch.tensor([100.0, 1.0, 5.0, 3.0, 4.0, 2.0])  # token 0 is skipped
    assert om.median_resid_norm(x) == 3.0
