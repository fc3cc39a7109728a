"""Error metric of the reference's parity harness (test infrastructure only).

rel_err follows tests/engine.mjs:17 of the reference: sqrt(sum (a - b)^2 / sum b^2) over the whole tensor.
Pinned by tests/test_oracle_metrics.py (closed forms).
"""
import torch


def rel_err(a, b):
    a = torch.as_tensor(a).detach().double().cpu()
    b = torch.as_tensor(b).detach().double().cpu()
    den = (b * b).sum()
    num = ((a - b) ** 2).sum()
    if float(den) == 0.0:
        return float(num.sqrt())
    return float((num / den).sqrt())


def max_abs(a, b):
    a = torch.as_tensor(a).detach().double().cpu()
    b = torch.as_tensor(b).detach().double().cpu()
    return float((a - b).abs().max()) if a.numel() else 0.0
