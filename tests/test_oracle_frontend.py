"""Pinning of oracle/frontend.py: library routines, closed forms and the already-pinned layer restatement."""
import math

import torch
import torch.nn.functional as F

from oracle import frontend as of
from oracle import model as om
from oracle.attention import apply_partial_rope, rope_inv_freq, rope_tables


def _y(B, T, Hk, dk, Hv, dv, extra, seed):
    g = torch.Generator().manual_seed(seed)
    C = 2 * Hk * dk + Hv * dv
    return torch.randn(B, T, C + extra, generator=g), C


def test_conv_matches_library_conv1d():
    """The causal depthwise conv + SiLU equals F.conv1d with left zero padding (HF:229-235 causal_conv1d_fn)."""
    B, T, Hk, dk, Hv, dv, K = 2, 9, 2, 8, 2, 8, 4
    y, C = _y(B, T, Hk, dk, Hv, dv, 2 * Hv, 0)
    w = torch.randn(C, K, generator=torch.Generator().manual_seed(1))
    bias = torch.randn(C, generator=torch.Generator().manual_seed(2))
    A_log, dt_bias = torch.zeros(Hv), torch.zeros(Hv)
    for b in (None, bias):
        q, k, v, _, _, _ = of.gdn_conv(y, w, None, A_log, dt_bias, Hk, dk, Hv, dv, C, C + Hv, conv_bias=b)
        ref = F.silu(F.conv1d(y[..., :C].transpose(1, 2), w[:, None, :], b, padding=K - 1, groups=C)[..., :T])
        ref = ref.transpose(1, 2)
        got = torch.cat([q.reshape(B, T, -1), k.reshape(B, T, -1), v.reshape(B, T, -1)], dim=-1)
        assert torch.allclose(got, ref, atol=1e-5, rtol=1e-5)


def test_conv_state_carries_across_calls():
    """Two calls (T1 then T2 tokens, state carried) give the outputs and final state of one call over T1 + T2."""
    B, Hk, dk, Hv, dv, K = 2, 1, 8, 1, 8, 4
    y, C = _y(B, 11, Hk, dk, Hv, dv, 2 * Hv, 3)
    w = torch.randn(C, K, generator=torch.Generator().manual_seed(4))
    A_log, dt_bias = torch.zeros(Hv), torch.zeros(Hv)
    full = of.gdn_conv(y, w, None, A_log, dt_bias, Hk, dk, Hv, dv, C, C + Hv)
    for split in (1, 2, 5):
        a = of.gdn_conv(y[:, :split], w, None, A_log, dt_bias, Hk, dk, Hv, dv, C, C + Hv)
        b = of.gdn_conv(y[:, split:], w, a[5], A_log, dt_bias, Hk, dk, Hv, dv, C, C + Hv)
        for i in range(3):
            assert torch.allclose(torch.cat([a[i], b[i]], dim=1), full[i], atol=1e-6)
        assert torch.allclose(b[5], full[5])
    # a state advanced by fewer than K-1 tokens keeps the older entries (shifted), as convState does
    one = of.gdn_conv(y[:, :1], w, full[5], A_log, dt_bias, Hk, dk, Hv, dv, C, C + Hv)
    assert torch.equal(one[5][:, :K - 2], full[5][:, 1:])
    assert torch.equal(one[5][:, K - 2], y[:, 0, :C])


def test_conv_unit_tap_is_a_shift():
    """Weight 1 on tap i, 0 elsewhere: the conv output at t is silu of the input at t - (K-1-i)."""
    B, T, Hk, dk, Hv, dv, K = 1, 7, 1, 4, 1, 4, 4
    y, C = _y(B, T, Hk, dk, Hv, dv, 2, 5)
    for i in range(K):
        w = torch.zeros(C, K)
        w[:, i] = 1.0
        q, k, v, *_ = of.gdn_conv(y, w, None, torch.zeros(1), torch.zeros(1), Hk, dk, Hv, dv, C, C + 1)
        got = torch.cat([q.reshape(B, T, -1), k.reshape(B, T, -1), v.reshape(B, T, -1)], dim=-1)
        lag = K - 1 - i
        exp = torch.zeros_like(got)
        exp[:, lag:] = F.silu(y[:, :T - lag, :C])
        assert torch.allclose(got, exp)


def test_gate_terms_and_softplus_threshold():
    B, T, Hk, dk, Hv, dv = 1, 3, 1, 4, 2, 4
    y, C = _y(B, T, Hk, dk, Hv, dv, 2 * Hv, 6)
    y[0, 0, C + Hv:] = torch.tensor([25.0, -3.0])   # a above the softplus threshold (20) and a moderate one
    A_log = torch.tensor([0.5, -1.0])
    dt_bias = torch.tensor([0.0, 0.25])
    _, _, _, g, beta, _ = of.gdn_conv(y, torch.zeros(C, 4), None, A_log, dt_bias, Hk, dk, Hv, dv, C, C + Hv)
    assert torch.allclose(beta, torch.sigmoid(y[..., C:C + Hv]))
    assert math.isclose(float(g[0, 0, 0]), -math.exp(0.5) * 25.0, rel_tol=1e-6)
    assert math.isclose(float(g[0, 0, 1]), -math.exp(-1.0) * math.log1p(math.exp(-2.75)), rel_tol=1e-6)


def test_gated_rmsnorm_closed_form():
    """A constant head vector c normalises to sign(c) (up to eps); the output is w * sign * silu(z) * scale."""
    Hv, dv = 2, 8
    o = torch.full((3, Hv, dv), 2.5)
    o[1] = -0.75
    z = torch.randn(3, Hv * dv, generator=torch.Generator().manual_seed(7))
    w = torch.randn(dv, generator=torch.Generator().manual_seed(8))
    hs = torch.tensor([2.0, -0.5])
    out = of.gated_rmsnorm(o, z, w, hs, eps=0.0).reshape(3, Hv, dv)
    sgn = torch.sign(o)
    exp = w * sgn * F.silu(z.reshape(3, Hv, dv)) * hs[:, None]
    assert torch.allclose(out, exp, atol=1e-6)


def test_attn_prep_matches_layer_pieces():
    """q / gate / k / v and the rotated keys equal the corresponding steps of oracle.model.attn_layer."""
    B, T, Hq, Hkv, D = 2, 5, 4, 2, 32
    g = torch.Generator().manual_seed(9)
    y = torch.randn(B, T, Hq * 2 * D + 2 * Hkv * D, generator=g)
    qw, kw = 0.1 * torch.randn(D, generator=g), 0.1 * torch.randn(D, generator=g)
    cos, sin = rope_tables(64, rope_inv_freq(D, 0.25, 1e7))
    pos = torch.tensor([0, 7])
    q, gate, k, v, k_rot = of.attn_prep(y, qw, kw, cos, sin, pos, Hq, Hkv, D)
    qg = y[..., :Hq * 2 * D].view(B, T, Hq, 2 * D)
    assert torch.equal(gate, qg[..., D:].reshape(B, T, Hq * D))
    assert torch.allclose(q, om.rmsnorm_1p(qg[..., :D], qw, 1e-6))
    kx = y[..., Hq * 2 * D:Hq * 2 * D + Hkv * D].view(B, T, Hkv, D)
    assert torch.allclose(k, om.rmsnorm_1p(kx, kw, 1e-6))
    assert torch.equal(v, y[..., Hq * 2 * D + Hkv * D:].view(B, T, Hkv, D))
    for b in range(B):
        p0 = int(pos[b])
        exp = apply_partial_rope(k[b:b + 1], cos[p0:p0 + T], sin[p0:p0 + T])[0]
        assert torch.allclose(k_rot[b], exp)
    # a planted mistake (positions not offset by pos) must be caught
    wrong = apply_partial_rope(k[1:2], cos[:T], sin[:T])[0]
    assert not torch.allclose(k_rot[1], wrong)
