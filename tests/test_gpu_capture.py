"""The MLP activation capture (the engine's `capture` hook, engine/model.js:9, :451-453: every neuron at every token
written by the `swiglu` kernel's `cap` binding, engine/kernels_qwen35.js:251-279) and the model-level hooks (`resid`
snapshots, per-head `heads` scales, neuron pushes) on the GPU.

Kernel level: the capture written by each SwiGLU epilogue equals, bitwise, the fp32 activations that epilogue
produces (the int8 GEMM's epilogues 2 and 3 on both of its kernels, the decode GEMV with and without its norm
prologue, q35_swiglu_push), lands at the strided [row, token] slots it is given and nowhere else, and leaves y
unchanged. Model level: the tiny stack's captured activations, residual snapshots, head-scaled and pushed runs
against the fp32 CPU oracle (itself pinned to HF's own down_proj pre-hook by tests/test_oracle_model.py)."""
import os
import sys

import pytest
import torch

import oracle
from oracle import mlp as omlp
from oracle import model as om
from q35hip import model as gm
from q35hip import ops
from gpu_util import announce, device

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
from tiny_weights import STEER_LAYER, tiny_config, tiny_inputs, tiny_weights  # noqa: E402

pytestmark = pytest.mark.gpu


def _gu(I, H, seed, gs):
    """Interleaved (gate, up) int8 rows with per-group (gs) or per-row scales."""
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(2 * I, H, generator=g) * 0.02
    if gs:
        return omlp.q8_quantize(w)
    s = w.abs().amax(dim=1) / 127.0
    return torch.clamp(torch.round(w / s[:, None]), -127, 127).to(torch.int8), s


def _slots(buf, t0, T):
    """The [rows, T, I] view a call of T tokens per row writes at token offset t0 of a [rows, capT, I] buffer."""
    return buf[:, t0:t0 + T]


def _untouched(buf, t0, T):
    rest = torch.cat([buf[:, :t0], buf[:, t0 + T:]], dim=1)
    return bool(torch.isnan(rest).all())


@pytest.mark.parametrize("M,T,I,gs,split", [(6144, 2048, 3584, True, True), (6144, 2048, 3584, False, False),
                                            (300, 100, 256, True, False), (90, 30, 512, False, True)])
def test_gemm_capture_equals_swiglu_output(M, T, I, gs, split):
    """The GEMM's SwiGLU epilogues (fp32 output and split output) write the same fp32 activations into the capture,
    bitwise equal to the fp32 epilogue's output: the DMA kernel with its row tail on the register-staged one (M 6144,
    I 3584, the stack's gate/up) and the register-staged kernel alone (small I), with pushes and 3 rows of T tokens
    written at token offset 5 of a longer capture buffer."""
    dev = device()
    H = 1024 if I == 3584 else 256
    q, s = _gu(I, H, M + I, gs)
    qd, sd = q.to(dev), s.to(dev)
    x = (torch.randn(M, H, generator=torch.Generator().manual_seed(M)) * 2.0).to(dev)
    pushes = ops.pack_pushes([(3, "mul", [2.0, -1.0, 0.5]), (None, "add", [0.25, 0.0, -0.25])], dev)
    rows, t0 = M // T, 5
    announce(f"gemm capture M{M} T{T} I{I} gs {gs} split {split}")
    a = ops.gemm_q8(x, qd, sd, epilogue="swiglu", pushes=pushes, T=T)
    cap = torch.full((rows, T + 9, I), float("nan"), device=dev)
    b = ops.gemm_q8(x, qd, sd, epilogue="swiglu", pushes=pushes, T=T, split_out=split, capture=_slots(cap, t0, T))
    torch.cuda.synchronize()
    assert torch.equal(_slots(cap, t0, T).reshape(M, I), a)
    assert _untouched(cap, t0, T)
    assert torch.equal(b, ops.split_activations(a) if split else a)


@pytest.mark.parametrize("M,gs,norm", [(3, True, True), (1, False, False), (8, True, False)])
def test_gemv_capture_equals_swiglu_output(M, gs, norm):
    """The decode GEMV's SwiGLU epilogue (with the residual add + RMSNorm prologue, and without) writes its
    activations into a [rows, 1, I] capture view, bitwise equal to its output."""
    dev = device()
    I, H = 3584, 1024
    q, s = _gu(I, H, 7 + M, gs)
    qd, sd = q.to(dev), s.to(dev)
    x = (torch.randn(M, H, generator=torch.Generator().manual_seed(M)) * 2.0).to(dev)
    pushes = ops.pack_pushes([(100, "add", [1.0, 2.0, 3.0]), (None, "mul", [0.5, 1.5, 2.0])], dev)
    pn = (None, torch.randn(H, generator=torch.Generator().manual_seed(2)).to(dev) * 0.1, 1e-6, None) if norm else None
    announce(f"gemv capture M{M} gs {gs} norm {norm}")
    a = ops.gemv(x, qd, sd, epilogue="swiglu", pushes=pushes, prenorm=pn)
    cap = torch.full((M, 3, I), float("nan"), device=dev)
    b = ops.gemv(x, qd, sd, epilogue="swiglu", pushes=pushes, prenorm=pn, capture=_slots(cap, 1, 1))
    torch.cuda.synchronize()
    assert torch.equal(b, a)
    assert torch.equal(cap[:, 1], a)
    assert _untouched(cap, 1, 1)


def test_swiglu_push_capture_equals_output():
    dev = device()
    M, T, I = 40, 20, 300
    gu = torch.randn(M, 2 * I, generator=torch.Generator().manual_seed(5)).to(dev)
    pushes = ops.pack_pushes([(7, "add", [1.0, -1.0])], dev)
    announce("swiglu_push capture")
    cap = torch.full((2, T + 2, I), float("nan"), device=dev)
    a = ops.swiglu_push(gu, pushes, T=T, capture=_slots(cap, 2, T))
    torch.cuda.synchronize()
    assert torch.equal(_slots(cap, 2, T).reshape(M, I), a)
    assert _untouched(cap, 2, T)


def test_capture_rejects_non_swiglu_epilogues_and_bad_views():
    dev = device()
    q, s = _gu(64, 256, 1, True)
    x = torch.randn(4, 256, device=dev)
    cap = torch.zeros(4, 1, 64, device=dev)
    with pytest.raises(RuntimeError):
        ops.gemv(x, q.to(dev), s.to(dev), epilogue="store", capture=cap)
    with pytest.raises(RuntimeError):
        ops.gemm_q8(x, q.to(dev), s.to(dev), epilogue="swiglu", capture=torch.zeros(4, 1, 63, device=dev))


def _tiny_pair(rows=2, **kw):
    cfg = tiny_config()
    W = tiny_weights(cfg)
    ids, vec = tiny_inputs(cfg)
    return cfg, W, ids[:rows], vec


def test_tiny_stack_capture_resid_against_oracle_and_logits_unchanged():
    """The tiny stack (3 GDN + 1 attention layers, steering after layer 1, a push on layer 2, head scales on layer
    0) with every hook on: the captured activations of every layer, the residual snapshots after each layer and after
    each mixer, and the logits of a 70-token prefill (in two calls of 40 + 30 tokens, filling one capture buffer
    through t0) and 4 decode steps match the fp32 CPU oracle; the prefill logits are bitwise those of a second model
    run without the capture. The MLP alone is also checked on the GPU's own residual: the captured activations equal the
    oracle's MLP activations of the snapshotted residual to 1e-5."""
    dev = device()
    cfg, W, ids, vec = _tiny_pair()
    L, I, H = cfg.layers, cfg.inter, cfg.hidden
    pushes = {2: [(5, "add", [0.75, -0.5]), (None, "mul", [1.25, 0.8])]}
    hs = {0: [0.5, 1.5]}
    announce("tiny stack capture / resid / heads / pushes")
    ref = om.OracleModel(cfg, W, steer_layer=STEER_LAYER)
    ref.set_vectors(torch.stack([vec, -vec]))
    ref.set_pushes(pushes)
    ref.set_head_scales(hs)
    lr, _ = ref.forward(ids, capture_layers=range(L))
    acts_r, resid_r, mix_r = dict(ref.acts), list(ref.resid_layer), list(ref.resid_mixer)

    def make():
        g = gm.HybridModel(cfg, W, dev, max_len=128, rows=2, steer_layer=STEER_LAYER)
        g.set_vectors(torch.stack([vec, -vec]), [0, 1])
        g.set_pushes(pushes)
        g.set_head_scales(hs)
        return g
    g, plain = make(), make()
    cap = torch.full((L, 2, 70, I), float("nan"), device=dev)
    res = torch.full((L, 2, 70, H), float("nan"), device=dev)
    mix = torch.full((L, 2, 70, H), float("nan"), device=dev)
    for a, b in ((0, 40), (40, 70)):
        # the mixer snapshots come from a second model run in step (same kernels, bitwise the same residual)
        lg, _ = g.forward(ids[:, a:b], capture=cap, resid=res, t0=a)
        lm, _ = plain.forward(ids[:, a:b], resid=mix, resid_mode="mixer", t0=a)
        assert torch.equal(lg, lm), "hooks changed the logits"
    torch.cuda.synchronize()
    assert not torch.isnan(cap).any() and not torch.isnan(res).any() and not torch.isnan(mix).any()
    assert oracle.rel_err(lg.cpu(), lr) <= 2e-2
    for l in range(L):
        ea = oracle.rel_err(cap[l].cpu(), acts_r[l])
        er = oracle.rel_err(res[l].cpu(), resid_r[l])
        em = oracle.rel_err(mix[l].cpu(), mix_r[l])
        # the MLP on the GPU's own residual: only the MLP's own arithmetic differs from the oracle's
        h = om.rmsnorm_1p(mix[l].cpu(), W[f"layers.{l}.post_attention_layernorm"], cfg.eps)
        own = om.mlp_act(W, l, h, pushes.get(l, ()))
        eo = oracle.rel_err(cap[l].cpu(), own)
        print(f"layer {l}: acts {ea:.2e} resid {er:.2e} mixer {em:.2e} acts on own resid {eo:.2e}")
        assert ea <= 2e-2 and er <= 2e-2 and em <= 2e-2
        assert eo <= 1e-5
    # decode: the step capture (eager) against the oracle's decode activations
    g.set_step_capture(list(range(L)))
    for step in range(4):
        nxt = lr.argmax(-1, keepdim=True)
        lr, _ = ref.forward(nxt, capture_layers=range(L))
        lg = g.decode_step(nxt.to(dev).reshape(2))
        torch.cuda.synchronize()
        assert oracle.rel_err(lg.cpu(), lr) <= 2e-2
        for l in range(L):
            e = oracle.rel_err(g.step_capture[l, :, 0].cpu(), ref.acts[l][:, 0])
            assert e <= 2e-2, (step, l, e)


def test_tiny_stack_decode_graph_capture_equals_eager_capture():
    """The decode graph records the step capture buffer: every replay's captured activations equal the eager step's
    (to the rounding of the split-K accumulations, which vary between runs)."""
    dev = device()
    cfg, W, ids, vec = _tiny_pair()
    L = cfg.layers
    announce("tiny stack decode graph capture")
    models = []
    for graph in (False, True):
        g = gm.HybridModel(cfg, W, dev, max_len=128, rows=2, steer_layer=STEER_LAYER)
        g.set_vectors(torch.stack([vec, -vec]), [0, 1])
        g.set_step_capture([0, 3])
        if graph:
            g.enable_decode_graph()
        models.append(g)
    eager, graph = models
    le, _ = eager.forward(ids)
    lg, _ = graph.forward(ids)
    assert torch.equal(le, lg)
    for step in range(5):
        nxt = le.argmax(-1)
        le = eager.decode_step(nxt).clone()
        ce = eager.step_capture.clone()
        lg = graph.decode_step(nxt).clone()
        cg = graph.step_capture.clone()
        torch.cuda.synchronize()
        assert oracle.rel_err(cg.cpu(), ce.cpu()) <= 1e-4, step
        assert oracle.rel_err(lg.cpu(), le.cpu()) <= 1e-4, step
    assert L == 4
