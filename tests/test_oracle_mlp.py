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
