"""Pinning of oracle/mlp.py."""
import torch

from oracle import mlp as omlp
from oracle import model as om


def test_q8_swiglu_equals_dequantised_layer_mlp():
    """The int8 SwiGLU path equals oracle.model.mlp on the same weights (dequantised once, as the HF fixture pins)."""
    g = torch.Generator().manual_seed(0)
    H, I = 64, 96
    W = {}
    for name, (n, k) in {"gate_proj": (I, H), "up_proj": (I, H), "down_proj": (H, I)}.items():
        W[f"layers.0.mlp.{name}.q"] = torch.randint(-127, 128, (n, k), generator=g, dtype=torch.int8)
        W[f"layers.0.mlp.{name}.s"] = torch.rand(n, generator=g) * 0.01
    key = "layers.0.mlp."
    x = torch.randn(5, H, generator=g)
    gg = omlp.q8_linear(x, W[key + "gate_proj.q"], W[key + "gate_proj.s"])
    uu = omlp.q8_linear(x, W[key + "up_proj.q"], W[key + "up_proj.s"])
    y = omlp.q8_linear(omlp.swiglu_push(gg, uu), W[key + "down_proj.q"], W[key + "down_proj.s"])
    Wm = {k.replace("layers.0.mlp.", "layers.0."): v for k, v in W.items()}
    assert torch.allclose(y, om.mlp(Wm, 0, x), atol=1e-5, rtol=1e-5)


def test_push_semantics_by_hand():
    g = torch.tensor([[0.0, 1.0, -1.0]] * 6)
    u = torch.ones(6, 3)
    base = torch.nn.functional.silu(g)
    # rows of 2 tokens each (T = 2): input rows 0-1 are sequence row 0, ..., rows 4-5 sequence row 2
    a = omlp.swiglu_push(g, u, [(1, "add", [10.0, 20.0, 30.0]), (1, "mul", [2.0]), (None, "mul", [1.0, 1.0, 0.5])],
                         T=2)
    exp = base.clone()
    for m in range(6):
        r = m // 2
        exp[m, 1] = (exp[m, 1] + [10.0, 20.0, 30.0][r]) * (2.0 if r == 0 else 1.0)
        exp[m] *= [1.0, 1.0, 0.5][r]
    assert torch.allclose(a, exp)
    # the row index is clamped to 3
    a = omlp.swiglu_push(torch.zeros(6, 1), torch.ones(6, 1), [(0, "add", [0.0, 1.0, 2.0, 3.0])], T=1)
    assert a[:, 0].tolist() == [0.0, 1.0, 2.0, 3.0, 3.0, 3.0]


def test_q8_quantize_closed_forms():
    """engine/kernels.js:15-47: a zero group gets scale 1 and zeros; a group holding integer multiples of c with
    max 127 c is reproduced exactly (scale c); a value at half a step rounds to the even neighbour."""
    N, K = 3, 256
    w = torch.zeros(N, K)
    c = 0.01
    w[1, 128:] = c * torch.arange(-127, 129)[:128].float().clamp(-127, 127)  # integer multiples, |max| 127 c
    w[2, :128] = torch.tensor([127.0] + [2.5] * 127)                      # scale 1: 2.5 -> 2 (half to even)
    q, s = omlp.q8_quantize(w)
    assert s.shape == (N, 2)
    assert s[0].tolist() == [1.0, 1.0] and int(q[0].abs().max()) == 0
    assert torch.allclose(s[1, 1], torch.tensor(c)) and torch.equal(q[1, 128:].float(), torch.round(w[1, 128:] / c))
    assert float(s[2, 0]) == 1.0 and q[2, 0] == 127 and bool((q[2, 1:128] == 2).all())


def test_q8_group_linear_matches_a_loop_over_groups():
    """q8_linear with group scales equals the sum over groups of (x_g . q_g) s_g, and the product quantizer is the
    oracle's restatement."""
    g = torch.Generator().manual_seed(3)
    w = torch.randn(5, 384, generator=g) * 0.05
    q, s = omlp.q8_quantize(w)
    from q35hip.workloads import quantize_groups_int8
    q2, s2 = quantize_groups_int8(w)
    assert torch.equal(q, q2) and torch.equal(s, s2)
    x = torch.randn(4, 384, generator=g, dtype=torch.float64)
    ref = torch.zeros(4, 5, dtype=torch.float64)
    for n in range(5):
        for gi in range(3):
            ref[:, n] += (x[:, 128 * gi:128 * gi + 128] @ q[n, 128 * gi:128 * gi + 128].double()) * float(s[n, gi])
    got = omlp.q8_linear(x.float(), q, s).double()
    assert float((got - ref).abs().max()) < 1e-5
    # quantization error is at most half a step of the group's scale
    err = (omlp.q8_dequant(q, s) - w).abs().reshape(5, 3, 128).amax(dim=2)
    assert bool((err <= s / 2 + 1e-7).all())
