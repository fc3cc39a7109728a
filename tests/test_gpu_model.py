"""The hybrid stack on the GPU (HIP hot path + torch glue) against the fp32 CPU oracle of the same weights."""
import os
import sys

import pytest
import torch

import oracle
import q35hip
from oracle import model as om
from q35hip import model as gm
from q35hip import workloads
from gpu_util import announce, device

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
from tiny_weights import STEER_LAYER, tiny_config, tiny_inputs, tiny_weights  # noqa: E402

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("gdn_prefill", ["recurrent", "chunk"])
def test_tiny_stack_prefill_decode_and_steering(gdn_prefill):
    dev = device()
    cfg = tiny_config()
    W = tiny_weights(cfg)
    ids, vec = tiny_inputs(cfg)
    announce(f"model tiny prefill/decode, GDN prefill {gdn_prefill}")
    ref = om.OracleModel(cfg, W, steer_layer=STEER_LAYER)
    ref.set_vectors(torch.stack([vec, -vec]))
    g = gm.HybridModel(cfg, W, dev, max_len=256, rows=2, steer_layer=STEER_LAYER, gdn_prefill=gdn_prefill)
    g.set_vectors(torch.stack([vec, -vec]), [0, 1])
    lr, _ = ref.forward(ids)
    lg, _ = g.forward(ids)
    assert oracle.rel_err(lg.cpu(), lr) <= 2e-2
    for _ in range(8):
        nxt = lr.argmax(-1, keepdim=True)
        lr, _ = ref.forward(nxt)
        lg, _ = g.forward(nxt.to(dev))
        assert oracle.rel_err(lg.cpu(), lr) <= 2e-2


def test_tiny_stack_rows_of_different_lengths_and_chunked_prefill():
    """The reference's steer loop prefills each row from its own prompt (reset(r); prefill(r, ...),
    engine/analysis.js:125) in chunks (engine/model.js:486-491), then decodes all rows together: rows of 37, 70 and 13
    tokens, row 1's prompt in chunks of 16, 32 and 22 tokens (multi-token calls over the KV cache), then 6 decode
    steps of all rows, each against its own single-row oracle."""
    dev = device()
    cfg = tiny_config()
    W = tiny_weights(cfg)
    ids, vec = tiny_inputs(cfg)
    prompts = [ids[0, :37], ids[1, :70], ids[0, 40:53]]
    announce("model tiny: rows of different lengths, chunked prefill")
    g = gm.HybridModel(cfg, W, dev, max_len=130, rows=3, steer_layer=STEER_LAYER)
    assert g.max_len % 64 == 0
    g.set_vectors(torch.stack([vec, -vec]), [0, -1, 1])
    refs, lr = [], []
    for r, pr in enumerate(prompts):
        ref = om.OracleModel(cfg, W, steer_layer=STEER_LAYER)
        ref.set_vectors([vec[None], None, -vec[None]][r] if r != 1 else torch.zeros(1, cfg.hidden))
        lr.append(ref.forward(pr[None])[0])
        refs.append(ref)
        g.reset(r)
        if r == 1:
            for a, b in ((0, 16), (16, 48), (48, 70)):
                lg, _ = g.forward(pr[a:b], row=r)
        else:
            lg, _ = g.forward(pr, row=r)
        assert oracle.rel_err(lg.cpu(), lr[r]) <= 2e-2, f"row {r} prefill"
    assert g.row_pos == [37, 70, 13]
    for step in range(6):
        nxt = torch.stack([l.argmax(-1) for l in lr])  # [3, 1]
        lg = g.decode_step(nxt.to(dev).reshape(3))
        lr = [refs[r].forward(nxt[r:r + 1])[0] for r in range(3)]
        for r in range(3):
            assert oracle.rel_err(lg[r:r + 1].cpu(), lr[r]) <= 2e-2, f"row {r} decode step {step}"


def test_tiny_stack_deterministic_decode_is_bitwise_repeatable():
    """deterministic=True: the decode step's residual adds sum in one fixed order, so a captured graph's replays and
    the eager steps of a second model give bitwise the same logits at every step (rows steered, 10 steps)."""
    dev = device()
    cfg = tiny_config()
    W = tiny_weights(cfg)
    ids, vec = tiny_inputs(cfg)
    announce("model tiny deterministic decode")
    eager = gm.HybridModel(cfg, W, dev, max_len=256, rows=2, steer_layer=STEER_LAYER, deterministic=True)
    graph = gm.HybridModel(cfg, W, dev, max_len=256, rows=2, steer_layer=STEER_LAYER, deterministic=True)
    graph.enable_decode_graph()
    for m in (eager, graph):
        m.set_vectors(torch.stack([vec, -vec]), [0, 1])
    le, _ = eager.forward(ids)
    lg, _ = graph.forward(ids)
    assert torch.equal(le, lg)
    for step in range(10):
        nxt = le.argmax(-1)
        le = eager.decode_step(nxt).clone()
        lg = graph.decode_step(nxt).clone()
        torch.cuda.synchronize()
        assert torch.equal(lg, le), f"replay {step} differs from eager"


def test_tiny_stack_decode_graph_replays_match_eager():
    """The captured decode step, replayed over 10 steps, gives the eager path's logits at every step (same kernels,
    same buffers), with eager work and synchronisations between the replays. The step's hidden-sized products split K
    and add their partial sums into the residual with fp32 atomics, so two runs of the same kernels agree to rounding
    (measured 2.4e-5 relative on these logits), not bit for bit: the bound is 1e-4."""
    dev = device()
    cfg = tiny_config()
    W = tiny_weights(cfg)
    ids, vec = tiny_inputs(cfg)
    announce("model tiny decode graph vs eager")
    eager = gm.HybridModel(cfg, W, dev, max_len=256, rows=2, steer_layer=STEER_LAYER)
    graph = gm.HybridModel(cfg, W, dev, max_len=256, rows=2, steer_layer=STEER_LAYER)
    graph.enable_decode_graph()
    for m in (eager, graph):
        m.set_vectors(torch.stack([vec, -vec]), [0, 1])
    le, _ = eager.forward(ids)
    lg, _ = graph.forward(ids)
    assert torch.equal(le, lg)
    for step in range(10):
        nxt = le.argmax(-1)
        le = eager.decode_step(nxt).clone()
        lg = graph.decode_step(nxt).clone()
        torch.cuda.synchronize()
        assert graph.pos == eager.pos
        assert oracle.rel_err(lg.cpu(), le.cpu()) <= 1e-4, f"replay {step} differs from eager"


_FULL_REF = {}
CAP_LAYERS = (0, 3, 11, 23)  # the layers of the reference's published activation check (README.md:156)
CAP_STEPS = 4                # decode steps whose activations the oracle keeps


def _full_weights(cfg, mlp_group):
    """Config-5 weights: the MLP int8 per output channel (mlp_group 0, the stated workload) or in the engine's
    group-128 format; the mixers, embedding and LM head in the engine's group-128 format either way."""
    return workloads.init_weights(cfg, seed=0, mlp_group=mlp_group)


def _full_stack_reference(cfg, W, prompt, steps, mlp_group):
    """The fp32 CPU oracle's steered greedy run of the full stack (computed once per MLP format and test module),
    with the MLP activations of CAP_LAYERS over the prefill and the first CAP_STEPS decode steps."""
    ref_d = _FULL_REF.get(mlp_group)
    if ref_d is None:
        announce(f"model full stack: CPU oracle (MLP group {mlp_group})")
        ref = om.OracleModel(cfg, W, steer_layer=12)
        _, resid = ref.forward(prompt[:1], collect_layer=12, stop_after=12)
        med = om.median_resid_norm(resid[0])
        v_ref = torch.randn(cfg.hidden, generator=torch.Generator().manual_seed(0))
        v_ref = v_ref / v_ref.norm() * (0.8 * med)
        ref.reset()
        ref.set_vectors(torch.stack([v_ref, torch.zeros_like(v_ref), -v_ref]))
        logits0, _ = ref.forward(prompt, capture_layers=CAP_LAYERS)
        acts_prefill = dict(ref.acts)
        toks, margins, acts_dec = [], [], []
        logits = logits0
        for i in range(steps):
            top2 = logits.topk(2, dim=-1)
            nxt = logits.argmax(dim=-1)
            toks.append(nxt)
            margins.append(top2.values[:, 0] - top2.values[:, 1])
            logits, _ = ref.forward(nxt[:, None], capture_layers=CAP_LAYERS if i < CAP_STEPS else ())
            if i < CAP_STEPS:
                acts_dec.append(dict(ref.acts))
        ref_d = dict(toks=torch.stack(toks, 1), margins=torch.stack(margins, 1), v=v_ref, prefill=logits0,
                     acts_prefill=acts_prefill, acts_decode=acts_dec)
        _FULL_REF[mlp_group] = ref_d
    return ref_d


@pytest.mark.timeout(1800)
@pytest.mark.parametrize("gdn_prefill,mlp_group", [("chunk", 0), ("recurrent", 0), ("chunk", 128),
                                                   ("recurrent", 128)])
def test_full_stack_steered_greedy_64_steps(gdn_prefill, mlp_group):
    """Qwen3.5-0.8B shape (24 layers, hidden 1024, SwiGLU 3584, tied 151,936 embedding), seed 0; batch 3,
    2048-token prompt (seed 0) on every row, vector after layer 12 scaled to 0.8 x the median residual norm: +v on
    row 0, none on row 1, -v on row 2; greedy tokens must be identical to the fp32 CPU path for 64 steps (decode
    steps replayed from a captured HIP graph). Run with the MLP int8 per output channel (the stated workload) and in
    the engine's group-128 format, and with each Gated DeltaNet prefill kernel: the chunked one (fp32 inputs: fp32
    products) and the token-serial one. The chunked per-channel case also runs the deterministic decode mode twice:
    both runs give the reference's tokens and bitwise the same top-2 margins."""
    dev = device()
    torch.set_num_threads(min(16, os.cpu_count() or 1))
    cfg = workloads.Q35Config()
    W = _full_weights(cfg, mlp_group)
    prompt = torch.randint(0, cfg.vocab, (1, 2048), generator=torch.Generator().manual_seed(0)).repeat(3, 1)
    steps = 64
    announce(f"model full stack: GPU (GDN prefill {gdn_prefill}, MLP group {mlp_group})")
    g = gm.HybridModel(cfg, W, dev, max_len=2048 + steps + 8, rows=3, gdn_prefill=gdn_prefill)
    g.enable_decode_graph()  # the 64 greedy steps replay one captured decode step
    toks_g, marg_g, v = gm.steered_greedy(g, prompt, steps)
    del g
    runs = []
    if gdn_prefill == "chunk" and mlp_group == 0:
        gd = gm.HybridModel(cfg, W, dev, max_len=2048 + steps + 8, rows=3, deterministic=True)
        gd.enable_decode_graph()
        for _ in range(2):
            runs.append(gm.steered_greedy(gd, prompt, steps)[:2])
        del gd
        assert torch.equal(runs[0][0], runs[1][0]) and torch.equal(runs[0][1], runs[1][1]), \
            "two deterministic runs differ"
    torch.cuda.empty_cache()
    ref_d = _full_stack_reference(cfg, W, prompt, steps, mlp_group)
    toks_r, marg_r, v_ref = ref_d["toks"], ref_d["margins"], ref_d["v"]
    assert oracle.rel_err(v, v_ref) <= 1e-3
    same = (toks_g == toks_r)
    first_diff = [int((~same[r]).nonzero()[0]) if not bool(same[r].all()) else -1 for r in range(3)]
    print(f"min top-2 margin (CPU) {float(marg_r.min()):.4g}; first differing step per row {first_diff}")
    assert bool(same.all()), f"greedy tokens differ; first differing step per row {first_diff}"
    for toks_d, _ in runs:
        assert torch.equal(toks_d, toks_r), "deterministic decode: greedy tokens differ from the CPU path"


@pytest.mark.timeout(1800)
def test_full_stack_prompt_prefilled_in_128_token_chunks_with_capture():
    """The config-5 workload (MLP int8 per output channel) with the 2048-token prompt prefilled in 16 calls of 128
    tokens (the engine's chunked prefill, engine/model.js:486-491: every call after the first attends over the KV
    cache), the MLP activations of layers 0, 3, 11 and 23 captured into one buffer through t0 (the engine's capture
    hook with capT0, engine/model.js:451-453, :486-491) and the residual after each mixer snapshotted: prefill logits
    within 2e-3 of the fp32 CPU path, the 64 greedy tokens of all three rows identical to it; the captured activations
    equal the oracle's MLP activations of the GPU's own snapshotted residual to 1e-4, and the oracle's end-to-end
    activations to within the stack's accumulated error (bf16 attention: 2e-2); the first 4 decode steps' captured
    activations (graph replays) likewise."""
    dev = device()
    torch.set_num_threads(min(16, os.cpu_count() or 1))
    cfg = workloads.Q35Config()
    W = _full_weights(cfg, 0)
    prompt = torch.randint(0, cfg.vocab, (1, 2048), generator=torch.Generator().manual_seed(0)).repeat(3, 1)
    steps = 64
    ref_d = _full_stack_reference(cfg, W, prompt, steps, 0)
    toks_r, v_ref = ref_d["toks"], ref_d["v"]
    announce("model full stack: prompt in 128-token chunks, capture at layers 0/3/11/23")
    g = gm.HybridModel(cfg, W, dev, max_len=2048 + steps + 8, rows=3)
    g.set_step_capture(CAP_LAYERS)
    g.enable_decode_graph()
    g.set_vectors(torch.stack([v_ref, -v_ref]), [0, -1, 1])
    cap = torch.zeros(len(CAP_LAYERS), 3, 2048, cfg.inter, device=dev)
    mix = torch.zeros(cfg.layers, 3, 2048, cfg.hidden, device=dev)
    for c in range(0, 2048, 128):
        logits, _ = g.forward(prompt[:, c:c + 128], capture=cap, capture_layers=CAP_LAYERS, resid=mix,
                              resid_mode="mixer", t0=c)
    e = oracle.rel_err(logits.cpu(), ref_d["prefill"])
    errs = []
    for i, l in enumerate(CAP_LAYERS):
        ce = cap[i].cpu()
        h = om.rmsnorm_1p(mix[l].cpu(), W[f"layers.{l}.post_attention_layernorm"], cfg.eps)
        e_own = oracle.rel_err(ce, om.mlp_act(W, l, h))
        e_ref = oracle.rel_err(ce, ref_d["acts_prefill"][l])
        errs.append((l, e_own, e_ref))
        assert e_own <= 1e-4, (l, e_own)
        assert e_ref <= 2e-2, (l, e_ref)
    del cap, mix
    toks, dec_errs = [], []
    for i in range(steps):
        nxt = q35hip.ops.argmax_rows(logits)
        toks.append(nxt.long().cpu())
        logits = g.decode_step(nxt)
        if i < CAP_STEPS:
            for j, l in enumerate(CAP_LAYERS):
                ed = oracle.rel_err(g.step_capture[j, :, 0].cpu(), ref_d["acts_decode"][i][l][:, 0])
                dec_errs.append(ed)
                assert ed <= 2e-2, (i, l, ed)
    toks_g = torch.stack(toks, 1)
    same = toks_g == toks_r
    first_diff = [int((~same[r]).nonzero()[0]) if not bool(same[r].all()) else -1 for r in range(3)]
    print(f"chunked prefill logits rel err {e:.3e}; activations (layer, own-resid err, end-to-end err) {errs}; "
          f"decode activations max err {max(dec_errs):.3e}; first differing step per row {first_diff}")
    assert e <= 2e-3
    assert bool(same.all()), f"greedy tokens differ; first differing step per row {first_diff}"


def test_loaded_int8_checkpoint_runs_on_the_stack(tmp_path):
    """A tiny HF-layout checkpoint loaded with every linear in int8 (q35hip.checkpoint) runs prefill and decode on
    the GPU stack in agreement with the oracle on the same loaded weights."""
    import test_checkpoint as tc
    from q35hip import checkpoint as ck
    dev = device()
    cfg0 = tiny_config()
    tc._write(str(tmp_path / "ckpt"), cfg0, tiny_weights(cfg0), shards=2)
    cfg, W = ck.load_checkpoint(str(tmp_path / "ckpt"))
    ids, _ = tiny_inputs(cfg)
    announce("model tiny loaded int8 checkpoint")
    ref = om.OracleModel(cfg, W)
    g = gm.HybridModel(cfg, W, dev, max_len=256, rows=2)
    lr, _ = ref.forward(ids)
    lg, _ = g.forward(ids)
    assert oracle.rel_err(lg.cpu(), lr) <= 2e-2
    for _ in range(4):
        nxt = lr.argmax(-1, keepdim=True)
        lr, _ = ref.forward(nxt)
        lg, _ = g.forward(nxt.to(dev))
        assert oracle.rel_err(lg.cpu(), lr) <= 2e-2
