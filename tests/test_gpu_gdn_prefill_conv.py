"""The GDN prefill with the front end in the chunk kernel's load phase (q35_gdn_chunk_prefill_conv: causal conv +
SiLU, l2 norms and gate terms computed while the chunk records are built) against the unfused pair (gdn_conv with
fp32 outputs, then the fp32 chunked rule) and the CPU oracle.

The fused kernels run the pair's arithmetic in the pair's order, so outputs, recurrent state and conv state are
compared bit for bit. Against the oracle (conv restated from HF:454-499, the fp32 recurrence of HF:331-380) the
fp32 bound of the chunked rule, relative error <= 1e-3; a prompt split over two calls carries both states and is
held to the same bound against the one-call result.
"""
import pytest
import torch

import oracle
from oracle import frontend as of
from q35hip import ops
from gpu_util import announce, device

pytestmark = pytest.mark.gpu

TOL_F32 = 1e-3


def _case(B, T, seed, Hk=16, H=16, d=128, K=4, bias=False):
    g = torch.Generator().manual_seed(seed)
    C = (2 * Hk + H) * d
    W = C + H * d + 2 * H  # [qkv | z | b | a], the fused projection row
    y = torch.randn(B, T, W, generator=g)
    conv_w = 0.5 * torch.randn(C, K, generator=g)
    cstate = torch.randn(B, K - 1, C, generator=g)
    A_log = torch.log(torch.rand(H, generator=g) * 16)
    dt_bias = torch.ones(H) + 0.1 * torch.randn(H, generator=g)
    S0 = 0.1 * torch.randn(B, H, d, d, generator=g)
    cb = torch.randn(C, generator=g) if bias else None
    return dict(y=y, conv_w=conv_w, cstate=cstate, A_log=A_log, dt_bias=dt_bias, S0=S0, cb=cb, C=C, W=W, Hk=Hk, H=H,
                d=d, b_off=C + H * d, a_off=C + H * d + H)


def _fused(c, dev, y=None, cstate=None, S=None):
    y = (c["y"] if y is None else y).to(dev).contiguous()
    cs = (c["cstate"] if cstate is None else cstate).to(dev).clone()
    S = (c["S0"] if S is None else S).to(dev).clone()
    o = ops.gdn_chunk_prefill_conv_(y, c["conv_w"].to(dev), cs, c["A_log"].to(dev), c["dt_bias"].to(dev), S,
                                    num_k_heads=c["Hk"], b_off=c["b_off"], a_off=c["a_off"],
                                    conv_bias=None if c["cb"] is None else c["cb"].to(dev))
    return o, S, cs


def _pair(c, dev):
    cs = c["cstate"].to(dev).clone()
    q, k, v, g, beta = ops.gdn_conv(c["y"].to(dev), c["conv_w"].to(dev), cs, c["A_log"].to(dev),
                                    c["dt_bias"].to(dev), num_k_heads=c["Hk"], head_k_dim=c["d"], num_v_heads=c["H"],
                                    head_v_dim=c["d"], b_off=c["b_off"], a_off=c["a_off"],
                                    conv_bias=None if c["cb"] is None else c["cb"].to(dev))
    o, S = ops.chunk_gated_delta_rule(q, k, v, g, beta, initial_state=c["S0"].to(dev), output_final_state=True,
                                      use_qk_l2norm_in_kernel=True)
    return o, S, cs


@pytest.mark.parametrize("B,T,Hk,bias", [(1, 1, 16, False), (2, 2, 16, True), (3, 5, 16, False),
                                         (2, 64, 16, True), (3, 65, 16, False), (2, 200, 4, True),
                                         (3, 2048, 16, False)])
def test_fused_front_end_equals_conv_then_chunk(B, T, Hk, bias):
    """Ragged lengths (one token, shorter than the conv window, one chunk, a chunk and one token, GQA with four k
    heads for 16 v heads) and the stack's B 3 T 2048 shape, with and without a conv bias, from non-zero conv and
    recurrent states: every output, the final state and the advanced conv state equal the unfused pair's."""
    dev = device()
    c = _case(B, T, seed=100 + T, Hk=Hk, bias=bias)
    announce(f"gdn chunk prefill conv B{B} T{T} Hk{Hk} bias {bias}")
    o_f, S_f, cs_f = _fused(c, dev)
    o_p, S_p, cs_p = _pair(c, dev)
    torch.cuda.synchronize()
    assert torch.equal(o_f.cpu(), o_p.cpu()), f"output: max diff {(o_f - o_p).abs().max().item():.3e}"
    assert torch.equal(S_f.cpu(), S_p.cpu()), f"state: max diff {(S_f - S_p).abs().max().item():.3e}"
    assert torch.equal(cs_f.cpu(), cs_p.cpu()), "conv state"


@pytest.mark.parametrize("T,Hk", [(37, 16), (130, 8)])
def test_fused_front_end_matches_oracle(T, Hk):
    """The fused call against the CPU oracle: the front end (conv state advanced to the last 3 inputs exactly, the
    conv and gate terms), then the fp32 recurrence from the initial state."""
    dev = device()
    B = 2
    c = _case(B, T, seed=200 + T, Hk=Hk, bias=True)
    announce(f"gdn chunk prefill conv vs oracle B{B} T{T} Hk{Hk}")
    o_f, S_f, cs_f = _fused(c, dev)
    torch.cuda.synchronize()
    q, k, v, g, beta, cs_r = of.gdn_conv(c["y"], c["conv_w"], c["cstate"], c["A_log"], c["dt_bias"], c["Hk"], c["d"],
                                         c["H"], c["d"], c["b_off"], c["a_off"], conv_bias=c["cb"])
    o_r, S_r = oracle.recurrent_gated_delta_rule(q, k, v, g, beta, initial_state=c["S0"], output_final_state=True,
                                                 use_qk_l2norm_in_kernel=True)
    eo, es = oracle.rel_err(o_f.cpu(), o_r), oracle.rel_err(S_f.cpu(), S_r)
    print(f"fused front end T{T} Hk{Hk}: rel err o {eo:.3e} S {es:.3e}")
    assert eo <= TOL_F32 and es <= TOL_F32
    assert torch.equal(cs_f.cpu(), cs_r)


def test_fused_front_end_prompt_in_two_calls():
    """A 150-token prompt as 70 + 80 tokens, conv and recurrent states carried on the device between the calls (the
    second call's first chunk reads the carried conv state), against the one-call result."""
    dev = device()
    B, T, T1 = 2, 150, 70
    c = _case(B, T, seed=300, bias=True)
    announce("gdn chunk prefill conv split 70 + 80")
    o_one, S_one, cs_one = _fused(c, dev)
    o_a, S_a, cs_a = _fused(c, dev, y=c["y"][:, :T1])
    o_b, S_b, cs_b = _fused(c, dev, y=c["y"][:, T1:], cstate=cs_a.cpu(), S=S_a.cpu())
    torch.cuda.synchronize()
    assert oracle.rel_err(torch.cat([o_a, o_b], dim=1).cpu(), o_one.cpu()) <= TOL_F32
    assert oracle.rel_err(S_b.cpu(), S_one.cpu()) <= TOL_F32
    assert torch.equal(cs_b.cpu(), cs_one.cpu())


def test_fused_front_end_rejects_other_conv_sizes():
    """Conv kernel sizes other than 4 are refused by the entry point (the layer then runs the unfused pair)."""
    dev = device()
    c = _case(1, 8, seed=400, K=3)
    with pytest.raises(RuntimeError):
        _fused(c, dev)
