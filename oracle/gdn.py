"""Gated delta rule, recurrent and chunked forms, on the CPU (test infrastructure only).

Restates HF:242-245 (l2norm), HF:331-380 (torch_recurrent_gated_delta_rule) and HF:249-327
(torch_chunk_gated_delta_rule) of transformers 5.15.0 models/qwen3_5/modeling_qwen3_5.py, which the reference's
PyTorch mirror (tests/engine_ref.py) runs; the WGSL `delta` kernel (engine/kernels_qwen35.js:209-236) computes the
same recurrence token by token.

One deliberate difference: HF applies the optional q/k l2norm in the input dtype before casting to fp32; here the
inputs are cast to the compute dtype first (identical for fp32 inputs, more precise for bf16 inputs). The HIP
kernels do the same.

Pinned (tests/test_oracle_gdn.py): the recurrence against the matrix (Householder) form of the gated delta rule
(Yang, Kautz, Hatamizadeh, ICLR 2025) computed independently in fp64, closed forms (beta = 0 gives pure decay;
g = 0, beta = 1, |k| = 1 writes v at key k; S = 0 gives o = (q.k) v), linearity in v; the chunked form against the
recurrence in fp64 for several T (including T not a multiple of the chunk), chunk sizes 16/32/64 and a non-zero
initial state.
"""
import math

import torch
import torch.nn.functional as F


def l2norm(x, dim=-1, eps=1e-6):
    """x * rsqrt(sum x^2 + eps) (HF:242-245; eps inside, not squared)."""
    return x * torch.rsqrt((x * x).sum(dim=dim, keepdim=True) + eps)


def _prep(query, key, value, g, beta, use_qk_l2norm_in_kernel, dtype):
    q, k, v, b, gg = [x.to(dtype) for x in (query, key, value, beta, g)]
    if use_qk_l2norm_in_kernel:
        q = l2norm(q)
        k = l2norm(k)
    H, Hk = v.shape[2], k.shape[2]
    if H != Hk:  # value heads outnumber q/k heads: repeat_interleave (HF:500-502)
        q = q.repeat_interleave(H // Hk, dim=2)
        k = k.repeat_interleave(H // Hk, dim=2)
    # [B, T, H, D] -> [B, H, T, D]
    return [x.transpose(1, 2).contiguous() for x in (q, k, v, b, gg)]


def recurrent_gated_delta_rule(query, key, value, g, beta, initial_state=None, output_final_state=True,
                               use_qk_l2norm_in_kernel=False, scale=None, dtype=torch.float32):
    """Token-serial gated delta rule (HF:331-380).

    query, key: [B, T, Hk, Dk]; value: [B, T, H, Dv]; g, beta: [B, T, H]; initial_state: [B, H, Dk, Dv] or None.
    Returns (o [B, T, H, Dv] in `dtype`, final state [B, H, Dk, Dv] in `dtype` or None).
    """
    q, k, v, b, gg = _prep(query, key, value, g, beta, use_qk_l2norm_in_kernel, dtype)
    B, H, T, Dk = k.shape
    Dv = v.shape[-1]
    scale = 1.0 / math.sqrt(Dk) if scale is None else scale
    q = q * scale
    S = torch.zeros(B, H, Dk, Dv, dtype=dtype) if initial_state is None else initial_state.to(dtype).clone()
    o = torch.zeros(B, H, T, Dv, dtype=dtype)
    for t in range(T):
        S = S * gg[:, :, t].exp()[..., None, None]
        kv_mem = (S * k[:, :, t, :, None]).sum(dim=-2)
        delta = (v[:, :, t] - kv_mem) * b[:, :, t, None]
        S = S + k[:, :, t, :, None] * delta[:, :, None, :]
        o[:, :, t] = (S * q[:, :, t, :, None]).sum(dim=-2)
    return o.transpose(1, 2).contiguous(), (S if output_final_state else None)


def chunk_gated_delta_rule(query, key, value, g, beta, chunk_size=64, initial_state=None, output_final_state=True,
                           use_qk_l2norm_in_kernel=False, scale=None, dtype=torch.float32):
    """Chunked gated delta rule (HF:249-327): zero-pad T to a multiple of chunk_size, cumulative gates per chunk,
    strictly-lower L = -(beta k k^T) * decay, forward substitution T = (I - L)^-1, U = T beta v,
    W = T beta exp(gamma) k, then the inter-chunk recurrence. Same arguments and returns as the recurrent form."""
    q, k, v, b, gg = _prep(query, key, value, g, beta, use_qk_l2norm_in_kernel, dtype)
    B, H, T, Dk = k.shape
    Dv = v.shape[-1]
    C = chunk_size
    pad = (C - T % C) % C
    q = F.pad(q, (0, 0, 0, pad))
    k = F.pad(k, (0, 0, 0, pad))
    v = F.pad(v, (0, 0, 0, pad))
    b = F.pad(b, (0, pad))
    gg = F.pad(gg, (0, pad))
    Tp = T + pad
    scale = 1.0 / math.sqrt(Dk) if scale is None else scale
    q = q * scale
    v_beta = v * b[..., None]
    k_beta = k * b[..., None]
    q, k, v, k_beta, v_beta = [x.reshape(B, H, -1, C, x.shape[-1]) for x in (q, k, v, k_beta, v_beta)]
    gg = gg.reshape(B, H, -1, C).cumsum(dim=-1)
    upper_incl = torch.triu(torch.ones(C, C, dtype=torch.bool), diagonal=0)
    decay = ((gg[..., :, None] - gg[..., None, :]).tril().exp()).tril()
    L = -((k_beta @ k.transpose(-1, -2)) * decay).masked_fill(upper_incl, 0)
    for i in range(1, C):
        row = L[..., i, :i].clone()
        sub = L[..., :i, :i].clone()
        L[..., i, :i] = row + (row[..., None] * sub).sum(-2)
    Tmat = L + torch.eye(C, dtype=dtype)
    u = Tmat @ v_beta
    w = Tmat @ (k_beta * gg.exp()[..., None])
    S = torch.zeros(B, H, Dk, Dv, dtype=dtype) if initial_state is None else initial_state.to(dtype).clone()
    o = torch.zeros_like(u)
    for c in range(Tp // C):
        qc, kc, uc = q[:, :, c], k[:, :, c], u[:, :, c]
        attn = qc @ kc.transpose(-1, -2) * decay[:, :, c]  # decay is lower-triangular incl. the diagonal
        v_new = uc - w[:, :, c] @ S
        o[:, :, c] = (qc * gg[:, :, c, :, None].exp()) @ S + attn @ v_new
        glast = gg[:, :, c, -1]
        S = S * glast.exp()[..., None, None] + (kc * (glast[..., None] - gg[:, :, c]).exp()[..., None]).transpose(
            -1, -2) @ v_new
    o = o.reshape(B, H, -1, Dv)[:, :, :T]
    return o.transpose(1, 2).contiguous(), (S if output_final_state else None)
