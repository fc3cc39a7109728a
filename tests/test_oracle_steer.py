"""Pins the steering add exactly. CPU only."""
import torch

import oracle


def test_rows_plus_none_minus_bitwise():
    x = torch.randn(3, 4, 8)
    v = torch.randn(8)
    out = oracle.residual_steer_add(x, torch.stack([v, -v]), torch.tensor([0, -1, 1]))
    assert torch.equal(out[0], x[0] + v) and torch.equal(out[1], x[1]) and torch.equal(out[2], x[2] - v)


def test_default_rows_clamp_like_wgsl():
    x = torch.zeros(6, 1, 2)
    vecs = torch.arange(8.0).view(4, 2)
    out = oracle.residual_steer_add(x, vecs, None)
    assert torch.equal(out[5, 0], vecs[3]) and torch.equal(out[2, 0], vecs[2])

