"""The SwiGLU MLP with int8 per-output-channel weights and the neuron hook, on the CPU (test infrastructure only).

Restates the engine's MLP path (engine/kernels.js:57-90 `matvec` over int8 weights; engine/kernels_qwen35.js:250-279
`swiglu`: a = silu(gate) * up, then each push of the layer in order, on its neuron or on every neuron, adds or
multiplies by its value for the row, the row index clamped to 3; the push records of engine/model.js:412-423) over
HF's Qwen3_5MLP (HF:704-717).

Pinned (tests/test_oracle_mlp.py): q8_linear against the dequantised fp32 product of oracle.model.mlp (which the HF
golden fixture pins), and the push semantics against hand-worked cases (add then multiply order, the all-neuron push,
the row clamp, tokens per row).
"""
import torch
import torch.nn.functional as F


def q8_linear(x, q, s):
    """x [M, K] fp32, q [N, K] int8, s [N] fp32 -> x @ (q * s)^T."""
    return x.float() @ (q.float() * s.float()[:, None]).T


def swiglu_push(g, u, pushes=(), T=1):
    """g, u: [M, I]; pushes: [(neuron or None, "add" | "mul", vals)] applied in order; row of input row m is
    min(m // T, 3)."""
    a = F.silu(g.float()) * u.float()
    M, I = a.shape
    for neuron, mode, vals in pushes:
        v = [float(x) for x in vals] + [1.0 if mode == "mul" else 0.0] * (4 - len(vals))
        rv = torch.tensor([v[min(m // T, 3)] for m in range(M)])[:, None]
        cols = slice(None) if neuron is None else slice(int(neuron), int(neuron) + 1)
        a[:, cols] = a[:, cols] * rv if mode == "mul" else a[:, cols] + rv
    return a
