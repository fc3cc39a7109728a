"""Residual steering add on the CPU (test infrastructure only).

Restates the layer-12 forward hook of the reference's tests/engine_ref.py:49-53 (layer output + s * vec at every
position, rows [+v, none, -v]) and the WGSL `resAdd` (engine/kernels.js:190-203: x[m, :] += v[min(row, 3), :]).
Pinned exactly (bitwise) by tests/test_oracle_steer.py against hand-built expectations.
"""
import torch


def residual_steer_add(x, vecs, vec_of_row=None):
    """x: [rows, T, H]; vecs: [nvec, H] fp32; vec_of_row: [rows] ints (negative = no vector) or None for
    min(row, nvec - 1). Returns a new tensor; the add is done in fp32 and rounded to x's dtype."""
    rows = x.shape[0]
    nvec = vecs.shape[0]
    out = x.clone()
    for r in range(rows):
        vi = min(r, nvec - 1) if vec_of_row is None else int(vec_of_row[r])
        if vi < 0:
            continue
        out[r] = (x[r].float() + vecs[vi].float()[None, :]).to(x.dtype)
    return out
