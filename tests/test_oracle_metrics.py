"""Pins the parity metric of the reference's harness (tests/engine.mjs:17: sqrt(sum (a - b)^2 / sum b^2) over the
whole tensor) with closed forms. CPU only."""
import math

import torch

import oracle
from oracle.metrics import max_abs


def test_rel_err_closed_forms():
    a = torch.tensor([3.0, 4.0])
    b = torch.tensor([0.0, 4.0])
    assert abs(oracle.rel_err(a, b) - 3.0 / 4.0) < 1e-12
    assert oracle.rel_err(b, b) == 0.0
    # scaling: a = (1 + e) b gives |e|, over any shape; a = -b gives 2
    x = torch.randn(3, 5, 7, generator=torch.Generator().manual_seed(0), dtype=torch.float64)
    assert abs(oracle.rel_err(1.01 * x, x) - 0.01) < 1e-9
    assert abs(oracle.rel_err(-x, x) - 2.0) < 1e-12
    # the error norm is over the whole tensor, not per element: one wrong entry of n equal ones gives 1 / sqrt(n)
    ones = torch.ones(16)
    bad = ones.clone()
    bad[5] = 2.0
    assert abs(oracle.rel_err(bad, ones) - 1.0 / math.sqrt(16)) < 1e-12
    # a zero reference reports the absolute norm of the difference
    assert abs(oracle.rel_err(torch.tensor([3.0, 4.0]), torch.zeros(2)) - 5.0) < 1e-12


def test_max_abs():
    assert max_abs(torch.tensor([1.0, -2.0, 3.0]), torch.tensor([1.5, 2.0, 3.0])) == 4.0
    assert max_abs(torch.zeros(0), torch.zeros(0)) == 0.0
