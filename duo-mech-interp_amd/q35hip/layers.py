"""Per-layer forward functions of the Qwen3.5 hybrid decoder, running the hot path on the q35:: HIP ops.

    gated_deltanet_layer(x, p, conv_state, rec_state, head_scale=None) -> y
    gated_attention_layer(x, p, k_cache, v_cache, pos) -> y
    residual_steer_add(x, vecs, rows) -> x

`p` holds one layer's weights under HF's parameter names (transformers 5.15.0 models/qwen3_5/modeling_qwen3_5.py,
HF:426-429 and HF:641-654; the engine's names at engine/model.js:89-112 map one to one):
  Gated DeltaNet   in_proj_qkv [C, H], in_proj_z [Hv*dv, H], in_proj_b [Hv, H], in_proj_a [Hv, H],
                   conv1d [C, K] (HF's [C, 1, K] is accepted), A_log [Hv], dt_bias [Hv], norm [dv], out_proj [H, Hv*dv]
  gated attention  q_proj [Hq*2*D, H] (per head [q | gate], HF:667-670), k_proj [Hkv*D, H], v_proj [Hkv*D, H],
                   o_proj [H, Hq*D], q_norm [D], k_norm [D]
States are caller-owned device tensors mutated in place, as the engine's buffers are (engine/model.js:308-342):
conv_state [B, K-1, C] fp32 (the last K-1 conv inputs, oldest first, engine/model.js:333), rec_state [B, Hv, dk, dv]
fp32, k_cache / v_cache [B, Hkv, max_len, D] bf16 holding rotated keys and values by position.

The glue (projections, depthwise causal conv, norms, gates) is torch on the device; the delta rule, the attention
and the steering add are the HIP kernels. Nothing here falls back to a CPU path: the ops raise on CPU tensors and
when the library is missing.
"""
import math

import torch
import torch.nn.functional as F

from . import ops

_ROPE_CACHE = {}


def rope_tables(n_pos, rot, theta, device):
    """cos / sin [n_pos, rot/2] fp32 of angle pos * theta^(-2j/rot) (HF:105-125 inv_freq in fp32, then the fp32
    product by position), cached per (n_pos, rot, theta, device)."""
    key = (int(n_pos), int(rot), float(theta), str(device))
    t = _ROPE_CACHE.get(key)
    if t is None:
        inv_freq = 1.0 / (theta ** (torch.arange(0, rot, 2, dtype=torch.int64).to(torch.float) / rot))
        ang = torch.arange(n_pos, dtype=torch.float32)[:, None] * inv_freq[None, :]
        t = (ang.cos().contiguous().to(device), ang.sin().contiguous().to(device))
        _ROPE_CACHE[key] = t
    return t


def rmsnorm_1p(x, w, eps=1e-6):
    """x * rsqrt(mean x^2 + eps) * (1 + w) in fp32 (HF:720-734; engine/kernels_qwen35.js:46-47)."""
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * (1.0 + w.float())).to(x.dtype)


def _rotate_rows(x, cos_rows, sin_rows):
    """Partial RoPE with rotate-half pairs (i, i + rot/2) on dims [0, rot) of x [B, T, H, D] (HF:546-589); the
    KV-cache writer's glue (the attention kernels rotate q and k themselves)."""
    half = cos_rows.shape[-1]
    rot = 2 * half
    c, s = cos_rows[None, :, None, :], sin_rows[None, :, None, :]
    x1, x2 = x[..., :half].float(), x[..., half:rot].float()
    return torch.cat([x1 * c - x2 * s, x2 * c + x1 * s, x[..., rot:].float()], dim=-1)


def gated_deltanet_layer(x, p, conv_state, rec_state, head_scale=None, *, num_k_heads=None, head_k_dim=None,
                         eps=1e-6, prefill="chunk"):
    """Gated DeltaNet mixer of one decoder layer (Qwen3_5GatedDeltaNet.forward, HF:432-543; the WGSL conv + delta
    kernels, engine/kernels_qwen35.js:127-247). x: [B, T, H] fp32 (the input-normed residual). A call with T == 1
    is one recurrent decode step (HF:505-517). T > 1 runs from rec_state either the chunked prefill (HF:518-530;
    prefill="chunk": bf16 MFMA products, relative error a few 1e-3) or the token-serial fp32 recurrence
    (prefill="recurrent": fp32 throughout, as the WGSL engine runs prefill token by token,
    engine/kernels_qwen35.js:183-247). Both states are updated in place. head_scale: optional [Hv] per-head output
    scale applied after the gated norm (engine/kernels_qwen35.js:243). num_k_heads / head_k_dim default to the
    value heads / value head dim (the Qwen3.5 text models use Hk = Hv and dk = dv). Returns y [B, T, H]."""
    if prefill not in ("chunk", "recurrent"):
        raise ValueError(f"gated_deltanet_layer: prefill must be 'chunk' or 'recurrent', not {prefill!r}")
    B, T, _ = x.shape
    Hv = p["A_log"].numel()
    dv = p["norm"].numel()
    Hk = Hv if num_k_heads is None else num_k_heads
    dk = dv if head_k_dim is None else head_k_dim
    kd = Hk * dk
    w = p["conv1d"]
    w = w.reshape(w.shape[0], w.shape[-1])
    K = w.shape[1]
    mixed = x @ p["in_proj_qkv"].T
    z = x @ p["in_proj_z"].T
    b = x @ p["in_proj_b"].T
    a = x @ p["in_proj_a"].T
    # depthwise causal conv over [carried K-1 inputs | this call's inputs], then SiLU (HF:199-240)
    full = torch.cat([conv_state.to(mixed.dtype), mixed], dim=1)
    conv = full[:, 0:T] * w[:, 0]
    for i in range(1, K):
        conv = conv + full[:, i:i + T] * w[:, i]
    conv = F.silu(conv)
    conv_state.copy_(full[:, T:T + K - 1])
    q = conv[..., :kd].reshape(B, T, Hk, dk).contiguous()
    k = conv[..., kd:2 * kd].reshape(B, T, Hk, dk).contiguous()
    v = conv[..., 2 * kd:].reshape(B, T, Hv, dv).contiguous()
    beta = torch.sigmoid(b).contiguous()
    g = (-p["A_log"].float().exp() * F.softplus(a.float() + p["dt_bias"].float())).contiguous()
    if T == 1 or prefill == "recurrent":
        o = ops.gdn_decode_step_(q, k, v, g, beta, rec_state, use_qk_l2norm_in_kernel=True)
    else:
        o, S = ops.chunk_gated_delta_rule(q, k, v, g, beta, initial_state=rec_state, output_final_state=True,
                                          use_qk_l2norm_in_kernel=True)
        rec_state.copy_(S)
    # gated RMSNorm: plain w, norm before the silu(z) gate (HF:168-184; engine/kernels_qwen35.js:237-243)
    o = o.reshape(B, T, Hv, dv)
    on = o * torch.rsqrt(o.pow(2).mean(-1, keepdim=True) + eps)
    o = (p["norm"] * on) * F.silu(z.reshape(B, T, Hv, dv))
    if head_scale is not None:
        o = o * head_scale.to(o.dtype)[:, None]
    return o.reshape(B, T, Hv * dv) @ p["out_proj"].T


def gated_attention_layer(x, p, k_cache, v_cache, pos, *, rope_theta=1e7, partial_rotary_factor=0.25, eps=1e-6,
                          cache_len=None):
    """Gated softmax attention mixer of one decoder layer (Qwen3_5Attention.forward, HF:656-701; WGSL attnPrep +
    attention, engine/kernels_qwen35.js:18-123). x: [B, T, H] fp32; the T tokens sit at positions pos..pos+T-1.
    Their rotated keys and values are written into the caches at those positions. T > 1 requires pos == 0 and runs
    the causal flash prefill over the call's own tokens; T == 1 runs the split-K decode over cache positions
    0..pos (cache_len: optional [B] int32 per-row lengths, default pos + 1). Returns y [B, T, H]."""
    B, T, _ = x.shape
    D = p["q_norm"].numel()
    Hq = p["q_proj"].shape[0] // (2 * D)
    Hkv = p["k_proj"].shape[0] // D
    rot = int(D * partial_rotary_factor)
    max_len = k_cache.shape[2]
    if pos + T > max_len:
        raise ValueError(f"gated_attention_layer: positions {pos}..{pos + T - 1} exceed the cache ({max_len})")
    cos, sin = rope_tables(max_len, rot, rope_theta, x.device)
    qg = (x @ p["q_proj"].T).view(B, T, Hq, 2 * D)
    q = rmsnorm_1p(qg[..., :D], p["q_norm"], eps)
    gate = qg[..., D:].reshape(B, T, Hq * D)
    k = rmsnorm_1p((x @ p["k_proj"].T).view(B, T, Hkv, D), p["k_norm"], eps)
    v = (x @ p["v_proj"].T).view(B, T, Hkv, D)
    k_cache[:, :, pos:pos + T] = _rotate_rows(k, cos[pos:pos + T], sin[pos:pos + T]).transpose(1, 2).to(k_cache.dtype)
    v_cache[:, :, pos:pos + T] = v.transpose(1, 2).to(v_cache.dtype)
    if T > 1:
        if pos != 0:
            raise ValueError("gated_attention_layer: a multi-token call must start at position 0")
        o = ops.gated_attention_prefill(q.to(torch.bfloat16).contiguous(), k.to(torch.bfloat16).contiguous(),
                                        v.to(torch.bfloat16).contiguous(), gate.to(torch.bfloat16).contiguous(),
                                        cos, sin, pos0=0, scale=1.0 / math.sqrt(D))
    else:
        cl = (torch.full((B,), pos + 1, dtype=torch.int32, device=x.device) if cache_len is None
              else cache_len.to(device=x.device, dtype=torch.int32))
        o = ops.gated_attention_decode(q[:, 0].to(torch.bfloat16).contiguous(), k_cache, v_cache,
                                       gate[:, 0].to(torch.bfloat16).contiguous(), cl, cos, sin,
                                       scale=1.0 / math.sqrt(D)).view(B, 1, Hq * D)
    return o.float() @ p["o_proj"].T


def residual_steer_add(x, vecs, rows=None):
    """x[r, t, :] += vecs[rows[r]] at every position t, in place (the layers[l] forward hook of
    tests/engine_ref.py:49-53 and the WGSL resAdd of engine/kernels.js:190-203). rows: [B] int, -1 for no vector;
    None gives row r the vector min(r, nvec - 1) as the WGSL's clamped row index does. Returns x."""
    if rows is not None and not torch.is_tensor(rows):
        rows = torch.as_tensor(rows, dtype=torch.int32, device=x.device)
    return ops.residual_steer_add_(x, vecs, rows)
