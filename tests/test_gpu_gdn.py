"""Gated DeltaNet parity on the GPU: HIP kernels against the CPU oracle (fp32 recurrence) on seeded inputs.

Tolerances (relative error sqrt(sum (a-b)^2 / sum b^2), the reference's metric, tests/engine.mjs:17):
  fp32 state with fp32 activations: <= 1e-3;  bf16 activations: <= 2e-2.
"""
import pytest
import torch

import oracle
import q35hip
from q35hip import workloads
from gpu_util import announce, device

pytestmark = pytest.mark.gpu

TOL_F32 = 1e-3
TOL_BF16 = 2e-2


def _oracle_rec(inp, state=None, dtype=torch.float32):
    return oracle.recurrent_gated_delta_rule(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"],
                                             initial_state=state, output_final_state=True,
                                             use_qk_l2norm_in_kernel=True, dtype=dtype)


def test_decode_64_sequential_steps_fp32():
    """64 sequential single-token decode steps, batch 1, 16 heads, d 128, fp32 state from 0, seed 0."""
    dev = device()
    inp = workloads.gdn_inputs(B=1, T=64, H=16, D=128, seed=0)
    o_ref, s_ref = _oracle_rec(inp)
    d = workloads.to_device(inp, dev)
    state = torch.zeros(1, 16, 128, 128, device=dev)
    outs = []
    announce("gdn decode 64 steps B1 H16 fp32")
    for t in range(64):
        sl = slice(t, t + 1)
        o = q35hip.gdn_decode_step_(d["q"][:, sl].contiguous(), d["k"][:, sl].contiguous(),
                                    d["v"][:, sl].contiguous(), d["g"][:, sl].contiguous(),
                                    d["beta"][:, sl].contiguous(), state)
        outs.append(o)
    o = torch.cat(outs, dim=1).cpu()
    torch.cuda.synchronize()
    assert oracle.rel_err(o, o_ref) <= TOL_F32
    assert oracle.rel_err(state.cpu(), s_ref) <= TOL_F32


def test_recurrent_long_prefill_fp32():
    """The token-serial kernel as a prefill: T = 2048 in one launch, B = 3, 16 heads, fp32 from a non-zero state
    (the hybrid stack's fp32 GDN prefill shape); fp32 tolerance."""
    dev = device()
    inp = workloads.gdn_inputs(B=3, T=2048, H=16, D=128, seed=3, dtype=torch.float32, normalize=False)
    s0 = 0.1 * torch.randn(3, 16, 128, 128, generator=torch.Generator().manual_seed(6))
    o_ref, s_ref = _oracle_rec(inp, s0)
    d = workloads.to_device(inp, dev)
    announce("gdn recurrent T2048 B3 H16 fp32")
    state = s0.to(dev)
    o = q35hip.gdn_decode_step_(d["q"], d["k"], d["v"], d["g"], d["beta"], state)
    torch.cuda.synchronize()
    assert oracle.rel_err(o.cpu(), o_ref) <= TOL_F32
    assert oracle.rel_err(state.cpu(), s_ref) <= TOL_F32


@pytest.mark.parametrize("regime", ["zero", "slow", "strong"])
def test_recurrent_gate_regimes_fp32(regime):
    """The token-serial kernel over T = 1024 in one launch with no decay (the state sums every token's update),
    slow decay, and decays that underflow e^g to 0: fp32 tolerance, finite outputs."""
    dev = device()
    inp = _gate_regime(workloads.gdn_inputs(B=1, T=1024, H=4, D=128, seed=37, dtype=torch.float32), regime, 37)
    o_ref, s_ref = _oracle_rec(inp)
    d = workloads.to_device(inp, dev)
    announce(f"gdn recurrent T1024 H4 fp32 gates {regime}")
    state = torch.zeros(1, 4, 128, 128, device=dev)
    o = q35hip.gdn_decode_step_(d["q"], d["k"], d["v"], d["g"], d["beta"], state)
    torch.cuda.synchronize()
    assert torch.isfinite(o).all() and torch.isfinite(state).all()
    eo, es = oracle.rel_err(o.cpu(), o_ref), oracle.rel_err(state.cpu(), s_ref)
    print(f"recurrent gates {regime}: rel err o {eo:.3e} S {es:.3e}")
    assert eo <= TOL_F32 and es <= TOL_F32


@pytest.mark.parametrize("B,H,Hk", [(16, 16, 16), (32, 8, 4)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_decode_step_many_states(B, H, Hk, dtype):
    """One token over B x H states (1024 blocks of 32 value columns), in place, from a non-zero state; the second
    shape has 8 value heads over 4 q/k heads."""
    dev = device()
    inp = workloads.gdn_inputs(B=B, T=1, H=H, Hk=Hk, D=128, seed=7, dtype=dtype, normalize=False)
    s0 = 0.1 * torch.randn(B, H, 128, 128, generator=torch.Generator().manual_seed(8))
    o_ref, s_ref = _oracle_rec(inp, s0)
    d = workloads.to_device(inp, dev)
    announce(f"gdn decode step B{B} H{H}/{Hk} {dtype}")
    state = s0.to(dev)
    o = q35hip.gdn_decode_step_(d["q"], d["k"], d["v"], d["g"], d["beta"], state)
    torch.cuda.synchronize()
    tol = TOL_F32 if dtype == torch.float32 else TOL_BF16
    assert oracle.rel_err(o.float().cpu(), o_ref) <= tol
    assert oracle.rel_err(state.cpu(), s_ref) <= tol
    # every (row, head) checked on its own, so that a unit written to the wrong place cannot hide in the norm
    err = ((state.cpu() - s_ref).flatten(2).norm(dim=2) / s_ref.flatten(2).norm(dim=2)).max().item()
    assert err <= tol


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_recurrent_multi_token_gqa_initial_state(dtype):
    """T = 37 in one launch, B = 2, 8 value heads over 4 q/k heads, a non-zero initial state."""
    dev = device()
    inp = workloads.gdn_inputs(B=2, T=37, H=8, Hk=4, D=128, seed=1, dtype=dtype, normalize=False)
    s0 = 0.1 * torch.randn(2, 8, 128, 128, generator=torch.Generator().manual_seed(5))
    o_ref, s_ref = _oracle_rec(inp, s0)
    d = workloads.to_device(inp, dev)
    announce(f"gdn recurrent T37 B2 H8/4 {dtype}")
    o, S = q35hip.recurrent_gated_delta_rule(d["q"], d["k"], d["v"], d["g"], d["beta"], initial_state=s0.to(dev),
                                             output_final_state=True, use_qk_l2norm_in_kernel=True)
    tol = TOL_F32 if dtype == torch.float32 else TOL_BF16
    assert oracle.rel_err(o.float().cpu(), o_ref) <= tol
    assert oracle.rel_err(S.cpu(), s_ref) <= tol


@pytest.mark.parametrize("T", [1, 63, 64, 65, 200])
def test_chunk_prefill_ragged_lengths(T):
    """Chunked prefill against the fp32 recurrence for T not a multiple of 64 (zero-padded tail), bf16 inputs."""
    dev = device()
    inp = workloads.gdn_inputs(B=2, T=T, H=4, D=128, seed=T, dtype=torch.bfloat16)
    o_ref, s_ref = _oracle_rec(inp)
    d = workloads.to_device(inp, dev)
    announce(f"gdn chunk T{T} B2 H4 bf16")
    o, S = q35hip.chunk_gated_delta_rule(d["q"], d["k"], d["v"], d["g"], d["beta"], output_final_state=True,
                                         use_qk_l2norm_in_kernel=True)
    assert oracle.rel_err(o.float().cpu(), o_ref) <= TOL_BF16
    assert oracle.rel_err(S.cpu(), s_ref) <= TOL_BF16


def _gate_regime(inp, regime, seed):
    """Rescale the generator's gates (g = -softplus(randn), about -0.8 per token: a 128-token pair decays by
    e^-100, so the state carried into a pair barely reaches its outputs) so that the carry matters: `zero` (no
    decay, the state accumulates over every pair), `slow` (x 0.03: about e^-3 per pair), `extreme` (slow, plus 2 %
    of the tokens at g = -1.2, a decay of e^-1.2 in one token), `strong` (x 10: e^gamma underflows to 0 inside a
    chunk; nothing may overflow)."""
    g = inp["g"]
    if regime == "zero":
        g = torch.zeros_like(g)
    elif regime == "slow":
        g = 0.03 * g
    elif regime == "extreme":
        hit = torch.rand(g.shape, generator=torch.Generator().manual_seed(seed)) < 0.02
        g = torch.where(hit, torch.full_like(g, -1.2), 0.02 * g)
    elif regime == "strong":
        g = 10.0 * g
    return dict(inp, g=g)


@pytest.mark.parametrize("regime", ["zero", "slow", "extreme", "strong"])
def test_chunk_prefill_gate_regimes_carry_across_pairs(regime):
    """bf16 chunked prefill over 8 pairs of 128 tokens with gates that let the state carry across the pair
    boundaries (the scan's e^G S + M S + Bm step and the output's Q' S term at full weight), and with gates strong
    enough to underflow the decay factors. Measured 2.4e-3 to 4.5e-3 on o and S."""
    dev = device()
    inp = _gate_regime(workloads.gdn_inputs(B=1, T=1024, H=4, D=128, seed=31, dtype=torch.bfloat16), regime, 31)
    o_ref, s_ref = _oracle_rec(inp)
    d = workloads.to_device(inp, dev)
    announce(f"gdn chunk T1024 H4 bf16 gates {regime}")
    o, S = q35hip.chunk_gated_delta_rule(d["q"], d["k"], d["v"], d["g"], d["beta"], output_final_state=True,
                                         use_qk_l2norm_in_kernel=True)
    assert torch.isfinite(o.float()).all() and torch.isfinite(S).all()
    eo, es = oracle.rel_err(o.float().cpu(), o_ref), oracle.rel_err(S.cpu(), s_ref)
    print(f"gates {regime}: rel err o {eo:.3e} S {es:.3e}")
    assert eo <= TOL_BF16 and es <= TOL_BF16


def test_chunk_prefill_no_decay_full_length():
    """No decay at all over T = 4096 (32 pairs): the final state is the whole sequence's delta-rule sum, so an error
    in the pair-to-pair chain accumulates into it. Measured 4.7e-3 (o), 3.9e-3 (S)."""
    dev = device()
    inp = _gate_regime(workloads.gdn_inputs(B=1, T=4096, H=4, D=128, seed=32, dtype=torch.bfloat16), "zero", 32)
    o_ref, s_ref = _oracle_rec(inp)
    d = workloads.to_device(inp, dev)
    announce("gdn chunk T4096 H4 bf16 no decay")
    o, S = q35hip.chunk_gated_delta_rule(d["q"], d["k"], d["v"], d["g"], d["beta"], output_final_state=True,
                                         use_qk_l2norm_in_kernel=True)
    eo, es = oracle.rel_err(o.float().cpu(), o_ref), oracle.rel_err(S.cpu(), s_ref)
    print(f"no decay T4096: rel err o {eo:.3e} S {es:.3e}")
    assert eo <= TOL_BF16 and es <= TOL_BF16


def test_chunk_prefill_long_sequence_slow_gates():
    """T = 32767 (256 pairs, a ragged last pair) with slow gates: the scan's pipelined pair loop over a long chain,
    the state carried across every boundary, against the fp32 recurrence."""
    dev = device()
    inp = _gate_regime(workloads.gdn_inputs(B=1, T=32767, H=2, D=128, seed=38, dtype=torch.bfloat16), "slow", 38)
    o_ref, s_ref = _oracle_rec(inp)
    d = workloads.to_device(inp, dev)
    announce("gdn chunk T32767 H2 bf16 slow gates")
    o, S = q35hip.chunk_gated_delta_rule(d["q"], d["k"], d["v"], d["g"], d["beta"], output_final_state=True,
                                         use_qk_l2norm_in_kernel=True)
    eo, es = oracle.rel_err(o.float().cpu(), o_ref), oracle.rel_err(S.cpu(), s_ref)
    print(f"T32767: rel err o {eo:.3e} S {es:.3e}")
    assert eo <= TOL_BF16 and es <= TOL_BF16


@pytest.mark.parametrize("regime", ["zero", "slow"])
def test_chunk_prefill_fp32_gate_regimes(regime):
    """The fp32 chunk path (the stack's) with the state carried across all 16 chunks of T = 1024: fp32 tolerance.
    Measured 3.5e-7 to 4.9e-7."""
    dev = device()
    inp = _gate_regime(workloads.gdn_inputs(B=1, T=1024, H=4, D=128, seed=36, dtype=torch.float32), regime, 36)
    o_ref, s_ref = _oracle_rec(inp)
    d = workloads.to_device(inp, dev)
    announce(f"gdn chunk T1024 H4 fp32 gates {regime}")
    o, S = q35hip.chunk_gated_delta_rule(d["q"], d["k"], d["v"], d["g"], d["beta"], output_final_state=True,
                                         use_qk_l2norm_in_kernel=True)
    eo, es = oracle.rel_err(o.cpu(), o_ref), oracle.rel_err(S.cpu(), s_ref)
    print(f"fp32 gates {regime}: rel err o {eo:.3e} S {es:.3e}")
    assert eo <= TOL_F32 and es <= TOL_F32


@pytest.mark.parametrize("B,T,H,Hk", [(3, 700, 5, 5), (2, 640, 8, 2)])
def test_chunk_prefill_slow_gates_initial_state_odd_shapes(B, T, H, Hk):
    """Slow gates with a non-zero initial state: B 3 x 5 heads (15 (row, head) units, not a multiple of 8: the scan's
    plain block order) over a ragged 6-pair sequence, and GQA (8 value heads over 2 q/k heads)."""
    dev = device()
    inp = _gate_regime(workloads.gdn_inputs(B=B, T=T, H=H, Hk=Hk, D=128, seed=33 + B, dtype=torch.bfloat16),
                       "slow", 33)
    s0 = 0.1 * torch.randn(B, H, 128, 128, generator=torch.Generator().manual_seed(34 + B))
    o_ref, s_ref = _oracle_rec(inp, s0)
    d = workloads.to_device(inp, dev)
    announce(f"gdn chunk B{B} T{T} H{H}/{Hk} bf16 slow gates, initial state")
    o, S = q35hip.chunk_gated_delta_rule(d["q"], d["k"], d["v"], d["g"], d["beta"], initial_state=s0.to(dev),
                                         output_final_state=True, use_qk_l2norm_in_kernel=True)
    eo, es = oracle.rel_err(o.float().cpu(), o_ref), oracle.rel_err(S.cpu(), s_ref)
    print(f"B{B} T{T} H{H}/{Hk}: rel err o {eo:.3e} S {es:.3e}")
    assert eo <= TOL_BF16 and es <= TOL_BF16


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_chunk_prefill_without_in_kernel_l2norm(dtype):
    """use_qk_l2norm_in_kernel=False on unit-norm q and k (the caller normalised them): both chunk paths against the
    recurrence without the in-kernel norm, slow gates."""
    dev = device()
    inp = _gate_regime(workloads.gdn_inputs(B=1, T=1024, H=4, D=128, seed=35, dtype=dtype), "slow", 35)
    o_ref, s_ref = oracle.recurrent_gated_delta_rule(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"],
                                                     output_final_state=True, use_qk_l2norm_in_kernel=False,
                                                     dtype=torch.float32)
    d = workloads.to_device(inp, dev)
    announce(f"gdn chunk T1024 H4 {dtype} without the in-kernel l2 norm")
    o, S = q35hip.chunk_gated_delta_rule(d["q"], d["k"], d["v"], d["g"], d["beta"], output_final_state=True,
                                         use_qk_l2norm_in_kernel=False)
    eo, es = oracle.rel_err(o.float().cpu(), o_ref), oracle.rel_err(S.cpu(), s_ref)
    print(f"no in-kernel l2 norm {dtype}: rel err o {eo:.3e} S {es:.3e}")
    tol = TOL_F32 if dtype == torch.float32 else TOL_BF16
    assert eo <= tol and es <= tol


def test_chunk_prefill_initial_state_and_gqa():
    dev = device()
    inp = workloads.gdn_inputs(B=1, T=256, H=8, Hk=2, D=128, seed=7, dtype=torch.bfloat16, normalize=False)
    s0 = 0.2 * torch.randn(1, 8, 128, 128, generator=torch.Generator().manual_seed(9))
    o_ref, s_ref = _oracle_rec(inp, s0)
    d = workloads.to_device(inp, dev)
    announce("gdn chunk T256 H8/2 initial state")
    o, S = q35hip.chunk_gated_delta_rule(d["q"], d["k"], d["v"], d["g"], d["beta"], initial_state=s0.to(dev),
                                         output_final_state=True, use_qk_l2norm_in_kernel=True)
    assert oracle.rel_err(o.float().cpu(), o_ref) <= TOL_BF16
    assert oracle.rel_err(S.cpu(), s_ref) <= TOL_BF16


@pytest.mark.parametrize("T", [1, 63, 64, 65, 300])
def test_chunk_prefill_fp32_inputs(T):
    """fp32 q/k/v take the fp32 chunk path: fp32 tolerance against the fp32 recurrence, ragged lengths."""
    dev = device()
    inp = workloads.gdn_inputs(B=1, T=T, H=4, D=128, seed=11 + T, dtype=torch.float32)
    o_ref, s_ref = _oracle_rec(inp)
    d = workloads.to_device(inp, dev)
    announce(f"gdn chunk T{T} fp32 inputs")
    o, S = q35hip.chunk_gated_delta_rule(d["q"], d["k"], d["v"], d["g"], d["beta"], output_final_state=True,
                                         use_qk_l2norm_in_kernel=True)
    assert o.dtype == torch.float32
    eo, es = oracle.rel_err(o.cpu(), o_ref), oracle.rel_err(S.cpu(), s_ref)
    print(f"fp32 chunk T{T}: rel err o {eo:.3e} S {es:.3e}")
    assert eo <= TOL_F32 and es <= TOL_F32


def test_chunk_prefill_fp32_stack_shape_gqa_initial_state():
    """The hybrid stack's GDN prefill shape on the fp32 chunk path: B = 3, T = 2048, 16 heads (a multiple of 8
    (row, head) units: the XCD-grouped block order), unnormalised fp32 inputs, non-zero initial state; plus a GQA
    case with 8 value heads over 2 q/k heads."""
    dev = device()
    for (B, T, H, Hk, seed) in ((3, 2048, 16, 16, 21), (2, 200, 8, 2, 22)):
        inp = workloads.gdn_inputs(B=B, T=T, H=H, Hk=Hk, D=128, seed=seed, dtype=torch.float32, normalize=False)
        s0 = 0.1 * torch.randn(B, H, 128, 128, generator=torch.Generator().manual_seed(seed + 100))
        o_ref, s_ref = _oracle_rec(inp, s0)
        d = workloads.to_device(inp, dev)
        announce(f"gdn chunk fp32 B{B} T{T} H{H}/{Hk} initial state")
        o, S = q35hip.chunk_gated_delta_rule(d["q"], d["k"], d["v"], d["g"], d["beta"], initial_state=s0.to(dev),
                                             output_final_state=True, use_qk_l2norm_in_kernel=True)
        eo, es = oracle.rel_err(o.cpu(), o_ref), oracle.rel_err(S.cpu(), s_ref)
        print(f"fp32 chunk B{B} T{T} H{H}/{Hk}: rel err o {eo:.3e} S {es:.3e}")
        assert eo <= TOL_F32 and es <= TOL_F32


def test_chunk_prefill_full_size():
    """B = 1, T = 4096, 16 heads, d 128, bf16 q/k/v, chunk 64, fp32 state; against the fp32 CPU recurrence."""
    dev = device()
    inp = workloads.gdn_inputs(B=1, T=4096, H=16, D=128, seed=0, dtype=torch.bfloat16)
    o_ref, s_ref = _oracle_rec(inp)
    d = workloads.to_device(inp, dev)
    announce("gdn chunk T4096 H16 bf16 (full size)")
    o, S = q35hip.chunk_gated_delta_rule(d["q"], d["k"], d["v"], d["g"], d["beta"], output_final_state=True,
                                         use_qk_l2norm_in_kernel=True)
    eo, es = oracle.rel_err(o.float().cpu(), o_ref), oracle.rel_err(S.cpu(), s_ref)
    print(f"T4096 rel err o {eo:.3e} S {es:.3e}")
    assert eo <= TOL_BF16 and es <= TOL_BF16


def test_chunk_then_decode_handoff():
    """Prefill 128 tokens with the chunk kernel, continue 16 tokens with the decode kernel on the carried state:
    equals one 144-token recurrence."""
    dev = device()
    inp = workloads.gdn_inputs(B=1, T=144, H=4, D=128, seed=3, dtype=torch.bfloat16)
    o_ref, s_ref = _oracle_rec(inp)
    d = workloads.to_device(inp, dev)
    announce("gdn chunk->decode handoff")
    pre = {k: v[:, :128].contiguous() for k, v in d.items()}
    o1, S = q35hip.chunk_gated_delta_rule(pre["q"], pre["k"], pre["v"], pre["g"], pre["beta"], output_final_state=True,
                                          use_qk_l2norm_in_kernel=True)
    outs = [o1]
    for t in range(128, 144):
        sl = slice(t, t + 1)
        outs.append(q35hip.gdn_decode_step_(d["q"][:, sl].contiguous(), d["k"][:, sl].contiguous(),
                                            d["v"][:, sl].contiguous(), d["g"][:, sl].contiguous(),
                                            d["beta"][:, sl].contiguous(), S))
    o = torch.cat(outs, dim=1).float().cpu()
    assert oracle.rel_err(o, o_ref) <= TOL_BF16
    assert oracle.rel_err(S.cpu(), s_ref) <= TOL_BF16
