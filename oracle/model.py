"""The Qwen3.5 hybrid decoder stack on the CPU in fp32 (test infrastructure only).

Restates the layer compositions that the reference's PyTorch mirror (tests/engine_ref.py) runs through transformers
5.15.0 models/qwen3_5/modeling_qwen3_5.py (HF:line), with the engine's layer loop (engine/model.js:404-466):
  rmsnorm_1p           HF:720-734 Qwen3_5RMSNorm: x * rsqrt(mean x^2 + eps) * (1 + w), in fp32
  rmsnorm_gated        HF:168-184 Qwen3_5RMSNormGated: plain w, norm before the silu(z) gate
  causal_conv          HF:199-239 depthwise causal conv (kernel 4) with carried state, then SiLU
  gdn_layer            HF:432-543 (in_proj_qkv / z / b / a, conv, split, beta, g, delta rule, gated norm, out_proj)
  attn_layer           HF:656-701 (q/gate interleave per head, q/k norm, partial RoPE, causal GQA, sigmoid gate)
  mlp                  HF:704-717 SwiGLU, here with int8 weights (per 128-input group or per row, dequantised
                       identically on the GPU path)
  decoder layer        HF:753-793 (pre-norm mixer + residual, pre-norm MLP + residual), plus the residual steering
                       add after one layer at every position (tests/engine_ref.py:49-53, engine/model.js:460)
  median residual norm engine/analysis.js:52-77 (median over tokens 1..T-1 of |x| after the layer)

The configuration object and the seeded weights come from the synthetic workload definition (q35hip.workloads
Q35Config / init_weights); this module only computes with them.

Pinned (tests/test_oracle_model.py) against golden vectors written by tests/golden/make_layer_golden.py from HF's own
Qwen3_5 modules on a tiny random config, and by invariants (decode continues prefill exactly, batch rows independent).
"""
import torch
import torch.nn.functional as F

from .attention import apply_partial_rope, rope_inv_freq, rope_tables
from .gdn import chunk_gated_delta_rule, recurrent_gated_delta_rule
from .mlp import q8_dequant, swiglu_push


def dequant(W, key):
    return q8_dequant(W[key + ".q"], W[key + ".s"])


# ------------------------------------------------------------------ pieces
def rmsnorm_1p(x, w, eps):
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * (1.0 + w.float())).to(x.dtype)


def rmsnorm_gated(x, z, w, eps):
    xf = x.float()
    xn = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return (w * xn.to(x.dtype) * F.silu(z.float())).to(x.dtype)


def causal_conv(x, w, state):
    """x: [B, T, C] (pre-conv), w: [C, K], state: [B, K-1, C] (previous inputs, oldest first) or None (zeros).
    Returns (silu(conv) [B, T, C], new state [B, K-1, C])."""
    B, T, C = x.shape
    K = w.shape[1]
    prev = torch.zeros(B, K - 1, C, dtype=x.dtype) if state is None else state
    full = torch.cat([prev, x], dim=1)  # [B, K-1+T, C]
    out = torch.zeros(B, T, C, dtype=x.dtype)
    for i in range(K):
        out = out + full[:, i:i + T, :] * w[:, i]
    return F.silu(out), full[:, -(K - 1):, :].clone()


def gdn_layer(cfg, W, l, h, state, decode, head_scale=None):
    """Gated DeltaNet mixer (HF:432-543). state: dict with 'conv' [B, K-1, C] and 'rec' [B, Hv, dk, dv] (or None).
    Prefill uses the chunked rule, decode (T == 1 with a state) the recurrent one, as HF:505-530 does. head_scale:
    optional [Hv] per-head output scale after the gated norm (engine/kernels_qwen35.js:243)."""
    p = f"layers.{l}."
    B, T, _ = h.shape
    mixed = h @ W[p + "in_proj_qkv"].T
    z = (h @ W[p + "in_proj_z"].T).reshape(B, T, cfg.lin_v_heads, cfg.lin_dv)
    b = h @ W[p + "in_proj_b"].T
    a = h @ W[p + "in_proj_a"].T
    conv_out, conv_state = causal_conv(mixed, W[p + "conv1d"], state.get("conv") if state else None)
    kd = cfg.lin_k_heads * cfg.lin_dk
    q = conv_out[..., :kd].reshape(B, T, cfg.lin_k_heads, cfg.lin_dk)
    k = conv_out[..., kd:2 * kd].reshape(B, T, cfg.lin_k_heads, cfg.lin_dk)
    v = conv_out[..., 2 * kd:].reshape(B, T, cfg.lin_v_heads, cfg.lin_dv)
    beta = torch.sigmoid(b)
    g = -W[p + "A_log"].float().exp() * F.softplus(a.float() + W[p + "dt_bias"])
    rec0 = state.get("rec") if state else None
    if decode:
        o, rec = recurrent_gated_delta_rule(q, k, v, g, beta, initial_state=rec0, output_final_state=True,
                                            use_qk_l2norm_in_kernel=True)
    else:
        o, rec = chunk_gated_delta_rule(q, k, v, g, beta, initial_state=rec0, output_final_state=True,
                                        use_qk_l2norm_in_kernel=True)
    o = rmsnorm_gated(o.reshape(-1, cfg.lin_dv), z.reshape(-1, cfg.lin_dv), W[p + "norm"], cfg.eps)
    if head_scale is not None:
        o = o.reshape(B, T, cfg.lin_v_heads, cfg.lin_dv) * head_scale.float()[:, None]
    y = o.reshape(B, T, -1) @ W[p + "out_proj"].T
    return y, {"conv": conv_state, "rec": rec}


def attn_layer(cfg, W, l, h, cache, pos, cos_t, sin_t):
    """Gated attention mixer (HF:656-701) over a KV cache holding rotated keys.
    cache: dict 'k', 'v' [B, Hkv, S, D] (keys / values of positions 0..pos-1) or None; the call's T tokens sit at
    positions pos..pos+T-1 and attend causally to the cache plus themselves."""
    p = f"layers.{l}."
    B, T, _ = h.shape
    D = cfg.head_dim
    qg = (h @ W[p + "q_proj"].T).view(B, T, cfg.n_heads, 2 * D)
    q, gate = qg[..., :D], qg[..., D:].reshape(B, T, cfg.n_heads * D)
    q = rmsnorm_1p(q, W[p + "q_norm"], cfg.eps)
    k = rmsnorm_1p((h @ W[p + "k_proj"].T).view(B, T, cfg.n_kv, D), W[p + "k_norm"], cfg.eps)
    v = (h @ W[p + "v_proj"].T).view(B, T, cfg.n_kv, D)
    cr, sr = cos_t[pos:pos + T], sin_t[pos:pos + T]
    q = apply_partial_rope(q, cr, sr)
    k = apply_partial_rope(k, cr, sr)
    kh, vh = k.transpose(1, 2), v.transpose(1, 2)
    if cache is not None:
        kh = torch.cat([cache["k"], kh], dim=2)
        vh = torch.cat([cache["v"], vh], dim=2)
    S = kh.shape[2]
    rep = cfg.n_heads // cfg.n_kv
    kr, vr = kh.repeat_interleave(rep, dim=1), vh.repeat_interleave(rep, dim=1)
    w = torch.matmul(q.transpose(1, 2), kr.transpose(2, 3)) * D ** -0.5
    qpos = torch.arange(pos, pos + T)[:, None]
    kpos = torch.arange(S)[None, :]
    w = w.masked_fill(kpos > qpos, float("-inf"))
    w = torch.softmax(w, dim=-1, dtype=torch.float32)
    o = torch.matmul(w, vr).transpose(1, 2).reshape(B, T, -1) * torch.sigmoid(gate)
    return o @ W[p + "o_proj"].T, {"k": kh, "v": vh}


def mlp_act(W, l, h, pushes=()):
    """The MLP activations silu(gate) * up (the down_proj input, where the engine's neuron hook sits) of h [B, T, H]
    (or [M, H], one token per row), with the layer's pushes applied (oracle.mlp.swiglu_push: the push row of token t
    of batch row b is min(b, 3))."""
    p = f"layers.{l}."
    T = h.shape[1] if h.dim() == 3 else 1
    g = (h @ dequant(W, p + "gate_proj").T).reshape(-1, W[p + "gate_proj.q"].shape[0])
    u = (h @ dequant(W, p + "up_proj").T).reshape(g.shape)
    return swiglu_push(g, u, pushes, T=T).reshape(*h.shape[:-1], -1)


def mlp(W, l, h, pushes=()):
    return mlp_act(W, l, h, pushes) @ dequant(W, f"layers.{l}.down_proj").T


class OracleModel:
    """fp32 CPU model with per-row recurrent states and KV caches; the steering add follows layer `steer_layer`."""

    def __init__(self, cfg, W, steer_layer=12):
        self.cfg, self.W, self.steer_layer = cfg, W, steer_layer
        self.cos, self.sin = rope_tables(1 << 15, rope_inv_freq(cfg.head_dim, cfg.partial_rotary, cfg.rope_theta))
        self.vecs = None
        self.pushes, self.head_scales = {}, {}
        self.reset()

    def reset(self):
        self.states = [None] * self.cfg.layers
        self.pos = 0

    def set_vectors(self, vecs):
        """vecs: [B, H] fp32 (zero rows for no vector), added after steer_layer at every position."""
        self.vecs = vecs

    def set_pushes(self, pushes):
        """{layer: [(neuron or None, "add" | "mul", [value per row])]}: the engine's neuron pushes
        (engine/model.js:412-423) at the down_proj input."""
        self.pushes = dict(pushes or {})

    def set_head_scales(self, scales):
        """{layer: [Hv] values}: per-head output scales of Gated DeltaNet layers (engine/model.js:362-368)."""
        self.head_scales = {l: torch.as_tensor(v, dtype=torch.float32) for l, v in (scales or {}).items()}

    def forward(self, ids, collect_layer=None, stop_after=None, capture_layers=()):
        """ids: [B, T] token ids continuing from self.pos. Returns (last-position logits [B, V] or None when
        stopping after layer stop_after, optional residual after collect_layer [B, T, H]). Also leaves, for the
        engine's hooks (engine/model.js:9-11): self.acts {layer: [B, T, I]} the MLP activations of capture_layers,
        self.resid_mixer / self.resid_layer [layers run] of [B, T, H] the residual after each mixer's residual add and
        after each layer."""
        cfg, W = self.cfg, self.W
        self.acts, self.resid_mixer, self.resid_layer = {}, [], []
        x = W["embed"][ids]
        T = ids.shape[1]
        decode = self.pos > 0 and T == 1
        collected = None
        last = cfg.layers - 1 if stop_after is None else stop_after
        for l in range(last + 1):
            p = f"layers.{l}."
            h = rmsnorm_1p(x, W[p + "input_layernorm"], cfg.eps)
            if cfg.is_attention(l):
                y, self.states[l] = attn_layer(cfg, W, l, h, self.states[l], self.pos, self.cos, self.sin)
            else:
                y, self.states[l] = gdn_layer(cfg, W, l, h, self.states[l], decode, self.head_scales.get(l))
            x = x + y
            self.resid_mixer.append(x)
            a = mlp_act(W, l, rmsnorm_1p(x, W[p + "post_attention_layernorm"], cfg.eps), self.pushes.get(l, ()))
            if l in capture_layers:
                self.acts[l] = a
            x = x + a @ dequant(W, p + "down_proj").T
            if l == self.steer_layer and self.vecs is not None:
                x = x + self.vecs[:, None, :]
            self.resid_layer.append(x)
            if l == collect_layer:
                collected = x.clone()
        self.pos += T
        if stop_after is not None:
            return None, collected
        hN = rmsnorm_1p(x[:, -1], W["norm"], cfg.eps)
        return hN @ W.get("lm_head", W["embed"]).T, collected


def median_resid_norm(resid):
    """Median over tokens 1..T-1 of |x_t| (engine/analysis.js:64-74: sort, take element len >> 1)."""
    n = resid[1:].norm(dim=-1).sort().values
    return float(n[n.shape[0] >> 1])


def greedy(model, prompt_ids, steps):
    """Prefill prompt_ids [B, T] then `steps` greedy tokens per row (argmax, lowest index on ties).
    Returns (tokens [B, steps], top-2 margins [B, steps])."""
    logits, _ = model.forward(prompt_ids)
    toks, margins = [], []
    for _ in range(steps):
        top2 = logits.topk(2, dim=-1)
        nxt = logits.argmax(dim=-1)
        toks.append(nxt)
        margins.append(top2.values[:, 0] - top2.values[:, 1])
        logits, _ = model.forward(nxt[:, None])
    return torch.stack(toks, 1), torch.stack(margins, 1)
