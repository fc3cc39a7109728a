"""The per-layer work around the two mixers, on the CPU (test infrastructure only).

Restates, over the fused projection output y (one row per token, the layout the engine's fused projection produces,
engine/kernels_qwen35.js:127-131):
  gdn_conv       HF:454-499 (causal_conv1d_fn / causal_conv1d_update at HF:199-239 with SiLU; split into q, k, v;
                 beta = sigmoid(b); g = -exp(A_log) * softplus(a + dt_bias)), and the WGSL conv / convState kernels
                 (engine/kernels_qwen35.js:133-178) with the gate terms of `delta` (:226-229; softplus threshold 20,
                 :11)
  gated_rmsnorm  HF:168-184 Qwen3_5RMSNormGated (norm in fp32, plain w, rounded to the input dtype before the weight
                 multiply) and the WGSL epilogue of `delta` (:237-243) with its per-head scale
  attn_prep      HF:667-680: per-head [q | gate] halves of q_proj, q_norm / k_norm (RMSNorm with 1 + w, HF:720-734),
                 RoPE of k at absolute positions and the cache update; WGSL attnPrep (engine/kernels_qwen35.js:18-69)

Pinned (tests/test_oracle_frontend.py): the conv against torch.nn.functional.conv1d (a library routine) and against
a one-call / two-call split of the same sequence (the carried state), a unit-tap kernel that must reproduce a pure
shift, softplus's threshold, the gated norm of a constant vector (closed form), and attn_prep against the pieces of
oracle.model.attn_layer (pinned end to end by the HF golden fixture).
"""
import torch
import torch.nn.functional as F

from .attention import apply_partial_rope
from .model import causal_conv, rmsnorm_1p, rmsnorm_gated


def gdn_conv(y, conv_w, conv_state, A_log, dt_bias, Hk, dk, Hv, dv, b_off, a_off, conv_bias=None):
    """y: [B, T, W] fp32; conv_w: [C, K]; conv_state: [B, K-1, C] or None (zeros). Returns
    (q [B, T, Hk, dk], k, v [B, T, Hv, dv], g [B, T, Hv], beta [B, T, Hv], new conv_state [B, K-1, C])."""
    B, T, _ = y.shape
    Kd, Vd = Hk * dk, Hv * dv
    C = 2 * Kd + Vd
    w = conv_w.reshape(C, -1).float()
    x = y[..., :C].float()
    if conv_bias is not None:
        # the bias enters before the SiLU, as F.conv1d's bias does (HF:216, :232)
        K = w.shape[1]
        prev = torch.zeros(B, K - 1, C) if conv_state is None else conv_state.float()
        full = torch.cat([prev, x], dim=1)
        pre = conv_bias.float() + sum(full[:, i:i + T, :] * w[:, i] for i in range(K))
        out, new_state = F.silu(pre), full[:, -(K - 1):, :].clone()
    else:
        out, new_state = causal_conv(x, w, None if conv_state is None else conv_state.float())
    q = out[..., :Kd].reshape(B, T, Hk, dk)
    k = out[..., Kd:2 * Kd].reshape(B, T, Hk, dk)
    v = out[..., 2 * Kd:].reshape(B, T, Hv, dv)
    beta = torch.sigmoid(y[..., b_off:b_off + Hv].float())
    g = -A_log.float().exp() * F.softplus(y[..., a_off:a_off + Hv].float() + dt_bias.float())
    return q, k, v, g, beta, new_state


def gated_rmsnorm(o, z, w, head_scale=None, eps=1e-6):
    """o: [..., Hv, dv] (fp32 or bf16); z: [..., Hv * dv]; w: [dv]. Returns [..., Hv * dv] in o's dtype."""
    Hv, dv = o.shape[-2], o.shape[-1]
    zz = z.reshape(*o.shape[:-2], Hv, dv)
    out = rmsnorm_gated(o, zz, w.float(), eps)
    if head_scale is not None:
        out = (out.float() * head_scale.float()[:, None]).to(o.dtype)
    return out.reshape(*o.shape[:-2], Hv * dv)


def attn_prep(y, q_norm_w, k_norm_w, cos_t, sin_t, pos, Hq, Hkv, D, eps=1e-6):
    """y: [B, T, W] fp32 holding [q_proj (Hq x [q | gate]) | k_proj | v_proj] per token; pos: [B] first positions.
    Returns (q [B, T, Hq, D] normalised, gate [B, T, Hq * D], k [B, T, Hkv, D] normalised (not rotated),
    v [B, T, Hkv, D], k_rot [B, T, Hkv, D] rotated at positions pos[b] + t), all fp32."""
    B, T, _ = y.shape
    qg = y[..., :Hq * 2 * D].reshape(B, T, Hq, 2 * D)
    q = rmsnorm_1p(qg[..., :D], q_norm_w, eps)
    gate = qg[..., D:].reshape(B, T, Hq * D)
    k = rmsnorm_1p(y[..., Hq * 2 * D:Hq * 2 * D + Hkv * D].reshape(B, T, Hkv, D), k_norm_w, eps)
    v = y[..., Hq * 2 * D + Hkv * D:Hq * 2 * D + 2 * Hkv * D].reshape(B, T, Hkv, D)
    k_rot = torch.stack([apply_partial_rope(k[b:b + 1], cos_t[int(pos[b]):int(pos[b]) + T],
                                            sin_t[int(pos[b]):int(pos[b]) + T])[0] for b in range(B)])
    return q, gate, k, v, k_rot
