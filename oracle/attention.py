"""Gated GQA softmax attention with partial RoPE, on the CPU (test infrastructure only).

Restates, from transformers 5.15.0 models/qwen3_5/modeling_qwen3_5.py:
  rope_inv_freq      HF:105-125 compute_default_rope_parameters (dim = int(head_dim * partial_rotary_factor))
  rope_tables        HF:129-147 rotary forward; for text every MRoPE stream carries the same positions, so the
                     interleave (HF:149-164) is the identity and cos/sin reduce to cos(pos * inv_freq)
  apply_partial_rope HF:546-589 rotate_half + apply_rotary_pos_emb on the first rot dims
  gated_attention    HF:656-698 (q/gate split left to the caller), eager_attention_forward HF:604-626 with the causal
                     mask, softmax in fp32, then * sigmoid(gate) (HF:698)
  gated_attention_cached  the same for T new tokens per row over a KV cache at per-row positions (HF:656-698 through
                     DynamicCache.update; the WGSL attention's key count n = pos + t + 1, engine/kernels_qwen35.js:90)
and the WGSL equivalents engine/kernels_qwen35.js:50-59 (rotation) and :73-123 (attention, gate).

Pinned (tests/test_oracle_attention.py): against torch.nn.functional.scaled_dot_product_attention (a library
routine) in fp64, against a brute-force per-query loop, RoPE closed forms (position 0 is the identity, each pair keeps
its norm, q.k after rotation depends only on the position difference, hand-computed pair rotation), decode equal to
the last prefill row, invariance of decode to how the context is split; the cached form against the self form
(position 0, cache = the call's rotated keys), against decode (T = 1), and a prompt split into two calls against one.
"""
import math

import torch


def rope_inv_freq(head_dim=256, partial_rotary_factor=0.25, theta=1e7):
    """inv_freq_j = 1 / theta^(2j / rot), j < rot/2, computed in fp32 as HF does (HF:123-124)."""
    rot = int(head_dim * partial_rotary_factor)
    return 1.0 / (theta ** (torch.arange(0, rot, 2, dtype=torch.int64).to(dtype=torch.float) / rot))


def rope_tables(n_pos, inv_freq):
    """cos, sin tables [n_pos, rot/2] in fp32: angle = pos * inv_freq (one fp32 product, as HF's fp32 matmul)."""
    pos = torch.arange(n_pos, dtype=torch.float32)
    ang = pos[:, None] * inv_freq[None, :].float()
    return ang.cos(), ang.sin()


def apply_partial_rope(x, cos_rows, sin_rows):
    """x: [..., T, H, D]; cos_rows/sin_rows: [T, rot/2] for the T positions of x. Rotates dims [0, rot) with
    rotate_half pairs (i, i + rot/2): out = x * cos + rotate_half(x) * sin; dims >= rot pass through."""
    half = cos_rows.shape[-1]
    rot = 2 * half
    if rot == 0:
        return x
    c = torch.cat([cos_rows, cos_rows], dim=-1).to(x.dtype)[:, None, :]  # [T, 1, rot]
    s = torch.cat([sin_rows, sin_rows], dim=-1).to(x.dtype)[:, None, :]
    xr, xp = x[..., :rot], x[..., rot:]
    x1, x2 = xr[..., :half], xr[..., half:]
    rh = torch.cat([-x2, x1], dim=-1)
    return torch.cat([xr * c + rh * s, xp], dim=-1)


def gated_attention(q, k, v, gate, cos_tab, sin_tab, pos0=0, scale=None, dtype=torch.float32):
    """Causal gated GQA attention over one call's tokens.

    q: [B, T, Hq, D]; k, v: [B, T, Hkv, D]; gate: [B, T, Hq * D]; cos_tab/sin_tab: [P, rot/2] (position pos0 + t).
    Returns [B, T, Hq * D] in `dtype`.
    """
    q, k, v, gate = [x.to(dtype) for x in (q, k, v, gate)]
    B, T, Hq, D = q.shape
    Hkv = k.shape[2]
    scale = D ** -0.5 if scale is None else scale
    if cos_tab is not None and cos_tab.shape[-1] > 0:
        cr, sr = cos_tab[pos0:pos0 + T].to(dtype), sin_tab[pos0:pos0 + T].to(dtype)
        q = apply_partial_rope(q, cr, sr)
        k = apply_partial_rope(k, cr, sr)
    qh = q.transpose(1, 2)  # [B, Hq, T, D]
    kh = k.transpose(1, 2).repeat_interleave(Hq // Hkv, dim=1)  # repeat_kv (HF:592-601)
    vh = v.transpose(1, 2).repeat_interleave(Hq // Hkv, dim=1)
    w = torch.matmul(qh, kh.transpose(2, 3)) * scale
    causal = torch.triu(torch.ones(T, T, dtype=torch.bool), diagonal=1)
    w = w.masked_fill(causal, float("-inf"))
    w = torch.softmax(w, dim=-1, dtype=dtype)
    o = torch.matmul(w, vh).transpose(1, 2).reshape(B, T, Hq * D)
    return o * torch.sigmoid(gate)


def gated_attention_decode(q, k_cache, v_cache, gate, cache_len, cos_tab, sin_tab, scale=None, dtype=torch.float32):
    """One query token per row over a KV cache of already-rotated keys.

    q: [B, Hq, D] (rotated here at position cache_len[b] - 1); k_cache, v_cache: [B, Hkv, max_len, D];
    gate: [B, Hq * D]; cache_len: [B] ints. Returns [B, Hq * D] in `dtype`.
    """
    q, k_cache, v_cache, gate = [x.to(dtype) for x in (q, k_cache, v_cache, gate)]
    B, Hq, D = q.shape
    Hkv = k_cache.shape[1]
    scale = D ** -0.5 if scale is None else scale
    out = torch.empty(B, Hq * D, dtype=dtype)
    for b in range(B):
        n = int(cache_len[b])
        qb = q[b][None]  # [1, Hq, D]
        if cos_tab is not None and cos_tab.shape[-1] > 0:
            qb = apply_partial_rope(qb, cos_tab[n - 1:n].to(dtype), sin_tab[n - 1:n].to(dtype))
        kb = k_cache[b, :, :n].repeat_interleave(Hq // Hkv, dim=0)  # [Hq, n, D]
        vb = v_cache[b, :, :n].repeat_interleave(Hq // Hkv, dim=0)
        w = torch.einsum("hd,hnd->hn", qb[0], kb) * scale
        w = torch.softmax(w, dim=-1, dtype=dtype)
        out[b] = torch.einsum("hn,hnd->hd", w, vb).reshape(-1)
    return out * torch.sigmoid(gate)


def gated_attention_cached(q, k_cache, v_cache, gate, pos, cos_tab, sin_tab, scale=None, dtype=torch.float32):
    """T new query tokens per row over a KV cache of already-rotated keys that holds them: token t of row b sits at
    position pos[b] + t (rotated there) and attends to cache keys 0 .. pos[b] + t.

    q: [B, T, Hq, D]; k_cache, v_cache: [B, Hkv, max_len, D]; gate: [B, T, Hq * D]; pos: [B] ints.
    Returns [B, T, Hq * D] in `dtype`.
    """
    q, k_cache, v_cache, gate = [x.to(dtype) for x in (q, k_cache, v_cache, gate)]
    B, T, Hq, D = q.shape
    Hkv = k_cache.shape[1]
    scale = D ** -0.5 if scale is None else scale
    out = torch.empty(B, T, Hq * D, dtype=dtype)
    for b in range(B):
        P = int(pos[b])
        qb = q[b:b + 1]
        if cos_tab is not None and cos_tab.shape[-1] > 0:
            qb = apply_partial_rope(qb, cos_tab[P:P + T].to(dtype), sin_tab[P:P + T].to(dtype))
        n = P + T
        kb = k_cache[b, :, :n].repeat_interleave(Hq // Hkv, dim=0)  # [Hq, n, D]
        vb = v_cache[b, :, :n].repeat_interleave(Hq // Hkv, dim=0)
        w = torch.matmul(qb[0].transpose(0, 1), kb.transpose(1, 2)) * scale  # [Hq, T, n]
        qpos = torch.arange(P, P + T)[:, None]
        w = w.masked_fill(torch.arange(n)[None, :] > qpos, float("-inf"))
        w = torch.softmax(w, dim=-1, dtype=dtype)
        out[b] = torch.matmul(w, vb).transpose(0, 1).reshape(T, Hq * D)
    return out * torch.sigmoid(gate)
