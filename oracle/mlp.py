"""The int8 weight format, the SwiGLU MLP with the neuron hook, on the CPU (test infrastructure only).

Restates the engine's q8 weights (engine/kernels.js:1-5, :15-47 `quantize`: one fp32 scale per group of 128 inputs of
a row, scale = max|w| / 127 or 1 for an all-zero group, q = round(w / scale)), its MLP path (engine/kernels.js:57-90
`matvec` over int8 weights; engine/kernels_qwen35.js:250-279 `swiglu`: a = silu(gate) * up, then each push of the
layer in order, on its neuron or on every neuron, adds or multiplies by its value for the row, the row index clamped
to 3; the push records of engine/model.js:412-423) over HF's Qwen3_5MLP (HF:704-717). Per-row scales ([N] instead of
[N, K / 128]) are accepted as well.

Pinned (tests/test_oracle_mlp.py): q8 quantization by closed forms (an all-zero group, a group whose values are
integer multiples of its scale, round half to even) and brute-force loops over groups; q8_linear against the
dequantised fp32 product of oracle.model.mlp (which the HF golden fixture pins) and against a per-group loop; the push
semantics against hand-worked cases (add then multiply order, the all-neuron push, the row clamp, tokens per row).
"""
import torch
import torch.nn.functional as F


def q8_quantize(w, group=128):
    """engine/kernels.js:15-47: w [N, K] -> (q [N, K] int8, s [N, K / group] fp32), per group of `group` inputs."""
    N, K = w.shape
    wg = w.float().reshape(N, K // group, group)
    m = wg.abs().amax(dim=2)
    s = torch.where(m == 0.0, torch.ones_like(m), m / 127.0)
    return torch.round(wg / s[:, :, None]).to(torch.int8).reshape(N, K), s


def q8_dequant(q, s):
    """fp32 weights of int8 q [N, K]: scales s [N, K / g] (one per group of g inputs) or [N] (one per row)."""
    if s.dim() == 1:
        return q.float() * s.float()[:, None]
    N, K = q.shape
    return (q.float().reshape(N, s.shape[1], K // s.shape[1]) * s.float()[:, :, None]).reshape(N, K)


def q8_linear(x, q, s):
    """x [M, K] fp32, q [N, K] int8, s [N] or [N, K / g] fp32 -> x @ dequant(q, s)^T."""
    return x.float() @ q8_dequant(q, s).T


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
