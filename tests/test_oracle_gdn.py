"""Pins the gated delta rule oracle (recurrent and chunked) without running the reference: the matrix form of the
rule computed independently in fp64, closed forms, and agreement of the two forms. CPU only."""
import pytest
import torch

import oracle
from q35hip import workloads


def matrix_form(q, k, v, g, beta, S0=None, scale=None):
    """Gated delta rule in the paper's matrix form (Yang, Kautz, Hatamizadeh, ICLR 2025), fp64, per head:
    M_t = alpha_t M_{t-1} (I - beta_t k_t k_t^T) + beta_t v_t k_t^T  with M [Dv, Dk];  o_t = M_t q_t.
    Inputs [B, T, H, D] already normalised; returns o [B, T, H, Dv] and the state transposed to [B, H, Dk, Dv]."""
    B, T, H, Dk = k.shape
    Dv = v.shape[-1]
    scale = Dk ** -0.5 if scale is None else scale
    q, k, v, g, beta = [x.double() for x in (q, k, v, g, beta)]
    o = torch.zeros(B, T, H, Dv, dtype=torch.float64)
    Sout = torch.zeros(B, H, Dk, Dv, dtype=torch.float64)
    I = torch.eye(Dk, dtype=torch.float64)
    for b in range(B):
        for h in range(H):
            M = torch.zeros(Dv, Dk, dtype=torch.float64) if S0 is None else S0[b, h].double().T.clone()
            for t in range(T):
                kt, vt = k[b, t, h], v[b, t, h]
                M = torch.exp(g[b, t, h]) * M @ (I - beta[b, t, h] * torch.outer(kt, kt)) + beta[b, t, h] * torch.outer(vt, kt)
                o[b, t, h] = M @ (q[b, t, h] * scale)
            Sout[b, h] = M.T
    return o, Sout


def test_recurrence_matches_matrix_form():
    inp = workloads.gdn_inputs(B=2, T=9, H=3, D=8, seed=0)
    S0 = 0.3 * torch.randn(2, 3, 8, 8, generator=torch.Generator().manual_seed(1))
    o, S = oracle.recurrent_gated_delta_rule(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], initial_state=S0,
                                             dtype=torch.float64)
    o2, S2 = matrix_form(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], S0)
    assert oracle.rel_err(o, o2) < 1e-12 and oracle.rel_err(S, S2) < 1e-12


def test_zero_beta_is_pure_decay():
    inp = workloads.gdn_inputs(B=1, T=1, H=2, D=16, seed=2)
    S0 = torch.randn(1, 2, 16, 16, generator=torch.Generator().manual_seed(3))
    _, S = oracle.recurrent_gated_delta_rule(inp["q"], inp["k"], inp["v"], inp["g"], torch.zeros_like(inp["beta"]),
                                             initial_state=S0, dtype=torch.float64)
    alpha = inp["g"][0, 0].double().exp()
    assert torch.allclose(S, S0.double() * alpha[None, :, None, None], atol=1e-12)


def test_unit_beta_no_decay_writes_v_at_k():
    """g = 0, beta = 1, |k| = 1: the updated state maps k to v exactly (S'^T k = v)."""
    inp = workloads.gdn_inputs(B=1, T=1, H=2, D=16, seed=4)
    S0 = torch.randn(1, 2, 16, 16, generator=torch.Generator().manual_seed(5))
    _, S = oracle.recurrent_gated_delta_rule(inp["q"], inp["k"], inp["v"], torch.zeros_like(inp["g"]),
                                             torch.ones_like(inp["beta"]), initial_state=S0, dtype=torch.float64)
    k, v = inp["k"][0, 0].double(), inp["v"][0, 0].double()
    got = torch.einsum("hkv,hk->hv", S[0], k)
    assert torch.allclose(got, v, atol=1e-10)


def test_zero_state_closed_form():
    """S = 0, beta = 1: o = (q . k) / sqrt(Dk) * v for the first token."""
    inp = workloads.gdn_inputs(B=1, T=1, H=2, D=32, seed=6)
    o, _ = oracle.recurrent_gated_delta_rule(inp["q"], inp["k"], inp["v"], inp["g"], torch.ones_like(inp["beta"]),
                                             dtype=torch.float64)
    q, k, v = [inp[n][0, 0].double() for n in ("q", "k", "v")]
    want = (q * k).sum(-1, keepdim=True) / 32 ** 0.5 * v
    assert torch.allclose(o[0, 0], want, atol=1e-12)


def test_linear_in_v_at_zero_state():
    inp = workloads.gdn_inputs(B=1, T=7, H=2, D=16, seed=7)
    v1 = inp["v"].double()
    v2 = torch.randn(v1.shape, generator=torch.Generator().manual_seed(70), dtype=torch.float64)
    a, _ = oracle.recurrent_gated_delta_rule(inp["q"], inp["k"], v1, inp["g"], inp["beta"], dtype=torch.float64)
    b, _ = oracle.recurrent_gated_delta_rule(inp["q"], inp["k"], v2, inp["g"], inp["beta"], dtype=torch.float64)
    c, _ = oracle.recurrent_gated_delta_rule(inp["q"], inp["k"], 2 * v1 - 3 * v2, inp["g"], inp["beta"],
                                             dtype=torch.float64)
    assert torch.allclose(c, 2 * a - 3 * b, atol=1e-10)


def test_l2norm_eps_inside():
    x = torch.tensor([[3.0, 4.0]], dtype=torch.float64)
    assert torch.allclose(oracle.l2norm(x), x / (25 + 1e-6) ** 0.5)


@pytest.mark.parametrize("T,C", [(1, 64), (63, 64), (64, 64), (65, 64), (200, 64), (100, 16), (100, 32)])
def test_chunk_equals_recurrence(T, C):
    inp = workloads.gdn_inputs(B=2, T=T, H=2, D=32, seed=T, normalize=False)
    S0 = 0.2 * torch.randn(2, 2, 32, 32, generator=torch.Generator().manual_seed(T))
    a = oracle.recurrent_gated_delta_rule(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], initial_state=S0,
                                          use_qk_l2norm_in_kernel=True, dtype=torch.float64)
    b = oracle.chunk_gated_delta_rule(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], chunk_size=C,
                                      initial_state=S0, use_qk_l2norm_in_kernel=True, dtype=torch.float64)
    assert oracle.rel_err(b[0], a[0]) < 1e-10 and oracle.rel_err(b[1], a[1]) < 1e-10


def test_gqa_value_heads_repeat_key_heads():
    """H = 2 Hk: value head h uses q/k head h // 2 (repeat_interleave, HF:500-502)."""
    inp = workloads.gdn_inputs(B=1, T=5, H=4, Hk=2, D=16, seed=9)
    o, _ = oracle.recurrent_gated_delta_rule(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], dtype=torch.float64)
    rep = {n: inp[n].repeat_interleave(2, dim=2) for n in ("q", "k")}
    o2, _ = oracle.recurrent_gated_delta_rule(rep["q"], rep["k"], inp["v"], inp["g"], inp["beta"], dtype=torch.float64)
    assert torch.allclose(o, o2)


def test_planted_transpose_is_caught():
    """A state-layout mistake (S[dv][dk] read instead of S[dk][dv]) changes the output: the matrix-form check above
    would fail for it. Planted in a copy of the inputs on the CPU."""
    inp = workloads.gdn_inputs(B=1, T=6, H=1, D=8, seed=11)
    S0 = torch.randn(1, 1, 8, 8, generator=torch.Generator().manual_seed(12))
    a, _ = oracle.recurrent_gated_delta_rule(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"], initial_state=S0,
                                             dtype=torch.float64)
    b, _ = oracle.recurrent_gated_delta_rule(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"],
                                             initial_state=S0.transpose(-1, -2), dtype=torch.float64)
    assert oracle.rel_err(a, b) > 1e-3
