"""Qwen3.5-shaped hybrid decoder stack on one MI355X: the hot path runs on the q35hip HIP ops, the glue around it
(projections, causal conv, norms, int8-dequantised SwiGLU, embedding, lm head) on torch.

Per-layer functions keep the reference's boundary: gated_deltanet_layer and gated_attention_layer are the mixers of
one decoder layer (HF: transformers 5.15.0 models/qwen3_5/modeling_qwen3_5.py, Qwen3_5GatedDeltaNet.forward HF:432-543
and Qwen3_5Attention.forward HF:656-701; engine/model.js:426-461 dispatches them per layer), and the residual
steering add after one layer mirrors the layers[12] forward hook of tests/engine_ref.py:49-53 and the WGSL resAdd
(engine/kernels.js:190-203). States are caller-owned tensors mutated in place (engine/model.js:333-336).
"""
import math

import torch
import torch.nn.functional as F

from . import ops


class Q35Weights:
    """Device copy of a weight dict (fp32; int8 MLP weights dequantised once, per output channel)."""

    def __init__(self, W, device):
        self.t = {}
        for k, v in W.items():
            if k.endswith(".q"):
                base = k[:-2]
                self.t[base] = (v.float() * W[base + ".s"][:, None]).to(device)
            elif k.endswith(".s"):
                continue
            else:
                self.t[k] = v.to(device)

    def __getitem__(self, k):
        return self.t[k]


def rmsnorm_1p(x, w, eps):
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * (1.0 + w.float())).to(x.dtype)


def rope_rows(x, cos_rows, sin_rows):
    """Rotate dims [0, rot) of x [B, T, H, D] with rotate_half pairs (glue for the KV-cache writer)."""
    half = cos_rows.shape[-1]
    rot = 2 * half
    c = cos_rows[None, :, None, :]
    s = sin_rows[None, :, None, :]
    x1, x2 = x[..., :half].float(), x[..., half:rot].float()
    return torch.cat([x1 * c - x2 * s, x2 * c + x1 * s, x[..., rot:].float()], dim=-1)


def gated_deltanet_layer(cfg, W, l, h, state, decode):
    """Gated DeltaNet mixer of layer l (HF:432-543). h: [B, T, H] fp32. state: dict with 'conv' [B, K-1, C] and
    'rec' [B, Hv, dk, dv] fp32 (mutated in place on decode), or None on a fresh prefill. Returns (y, state)."""
    p = f"layers.{l}."
    B, T, _ = h.shape
    mixed = h @ W[p + "in_proj_qkv"].T
    z = h @ W[p + "in_proj_z"].T
    b = h @ W[p + "in_proj_b"].T
    a = h @ W[p + "in_proj_a"].T
    w = W[p + "conv1d"]
    K = w.shape[1]
    prev = torch.zeros(B, K - 1, mixed.shape[-1], device=h.device) if state is None else state["conv"]
    full = torch.cat([prev, mixed], dim=1)
    conv = full[:, 0:T] * w[:, 0]
    for i in range(1, K):
        conv = conv + full[:, i:i + T] * w[:, i]
    conv = F.silu(conv)
    new_conv = full[:, -(K - 1):].contiguous()
    kd = cfg.lin_k_heads * cfg.lin_dk
    q = conv[..., :kd].reshape(B, T, cfg.lin_k_heads, cfg.lin_dk).contiguous()
    k = conv[..., kd:2 * kd].reshape(B, T, cfg.lin_k_heads, cfg.lin_dk).contiguous()
    v = conv[..., 2 * kd:].reshape(B, T, cfg.lin_v_heads, cfg.lin_dv).contiguous()
    beta = torch.sigmoid(b).contiguous()
    g = (-W[p + "A_log"].exp() * F.softplus(a + W[p + "dt_bias"])).contiguous()
    if decode:
        rec = state["rec"]
        o = ops.gdn_decode_step_(q, k, v, g, beta, rec, use_qk_l2norm_in_kernel=True)
    else:
        rec0 = None if state is None else state["rec"]
        o, rec = ops.chunk_gated_delta_rule(q, k, v, g, beta, initial_state=rec0, output_final_state=True,
                                            use_qk_l2norm_in_kernel=True)
    o = o.reshape(-1, cfg.lin_dv)
    on = o * torch.rsqrt(o.pow(2).mean(-1, keepdim=True) + cfg.eps)
    o = (W[p + "norm"] * on) * F.silu(z.reshape(-1, cfg.lin_dv))
    return o.reshape(B, T, -1) @ W[p + "out_proj"].T, {"conv": new_conv, "rec": rec}


def gated_attention_layer(cfg, W, l, h, cache, pos, cos, sin):
    """Gated attention mixer of layer l (HF:656-701). cache: dict 'k', 'v' bf16 [B, Hkv, max_len, D] (rotated keys),
    filled here for positions pos..pos+T-1. Prefill (pos == 0) runs the fused RoPE + causal flash kernel; decode
    (T == 1) the split-K kernel over the cache."""
    p = f"layers.{l}."
    B, T, _ = h.shape
    D = cfg.head_dim
    qg = (h @ W[p + "q_proj"].T).view(B, T, cfg.n_heads, 2 * D)
    q = rmsnorm_1p(qg[..., :D], W[p + "q_norm"], cfg.eps)
    gate = qg[..., D:].reshape(B, T, cfg.n_heads * D)
    k = rmsnorm_1p((h @ W[p + "k_proj"].T).view(B, T, cfg.n_kv, D), W[p + "k_norm"], cfg.eps)
    v = (h @ W[p + "v_proj"].T).view(B, T, cfg.n_kv, D)
    k_rot = rope_rows(k, cos[pos:pos + T], sin[pos:pos + T])
    cache["k"][:, :, pos:pos + T] = k_rot.transpose(1, 2).to(torch.bfloat16)
    cache["v"][:, :, pos:pos + T] = v.transpose(1, 2).to(torch.bfloat16)
    if T > 1:
        if pos != 0:
            raise ValueError("gated_attention_layer: multi-token calls continue from position 0 only")
        o = ops.gated_attention_prefill(q.to(torch.bfloat16).contiguous(), k.to(torch.bfloat16).contiguous(),
                                        v.to(torch.bfloat16).contiguous(), gate.to(torch.bfloat16).contiguous(),
                                        cos, sin, pos0=pos)
    else:
        cl = torch.full((B,), pos + 1, dtype=torch.int32, device=h.device)
        o = ops.gated_attention_decode(q[:, 0].to(torch.bfloat16).contiguous(), cache["k"], cache["v"],
                                       gate[:, 0].to(torch.bfloat16).contiguous(), cl, cos, sin).view(B, 1, -1)
    return o.float() @ W[p + "o_proj"].T


def mlp(W, l, h):
    p = f"layers.{l}."
    return (F.silu(h @ W[p + "gate_proj"].T) * (h @ W[p + "up_proj"].T)) @ W[p + "down_proj"].T


class HybridModel:
    """B independent rows decoded together (the boosted / as-is / suppressed rows of the reference's steer loop,
    engine/analysis.js:117-145). fp32 residual stream; vectors added after steer_layer at every position."""

    def __init__(self, cfg, W, device, max_len=4096, rows=3, steer_layer=12):
        self.cfg, self.device, self.steer_layer = cfg, device, steer_layer
        self.W = W if isinstance(W, Q35Weights) else Q35Weights(W, device)
        rot = int(cfg.head_dim * cfg.partial_rotary)
        inv_freq = 1.0 / (cfg.rope_theta ** (torch.arange(0, rot, 2, dtype=torch.int64).to(torch.float) / rot))
        ang = torch.arange(max_len, dtype=torch.float32)[:, None] * inv_freq[None, :]
        self.cos, self.sin = ang.cos().contiguous().to(device), ang.sin().contiguous().to(device)
        self.max_len, self.rows = max_len, rows
        self.vecs = None
        self.vec_rows = None
        self.caches = {}
        for l in range(cfg.layers):
            if cfg.is_attention(l):
                shape = (rows, cfg.n_kv, max_len, cfg.head_dim)
                self.caches[l] = {"k": torch.zeros(shape, dtype=torch.bfloat16, device=device),
                                  "v": torch.zeros(shape, dtype=torch.bfloat16, device=device)}
        self.reset()

    def reset(self):
        self.states = [None] * self.cfg.layers
        self.pos = 0

    def set_vectors(self, vecs, vec_of_row):
        """vecs: [n, H] fp32; vec_of_row: [rows] int (-1 = no vector)."""
        self.vecs = vecs.to(self.device, torch.float32).contiguous()
        self.vec_rows = torch.as_tensor(vec_of_row, dtype=torch.int32).to(self.device)

    @torch.no_grad()
    def forward(self, ids, stop_after=None, collect_layer=None):
        cfg, W = self.cfg, self.W
        T = ids.shape[1]
        if self.pos + T > self.max_len:
            raise ValueError("context exceeds the KV cache")
        x = W["embed"][ids.to(self.device)]
        decode = self.pos > 0 and T == 1
        collected = None
        last = cfg.layers - 1 if stop_after is None else stop_after
        for l in range(last + 1):
            p = f"layers.{l}."
            h = rmsnorm_1p(x, W[p + "input_layernorm"], cfg.eps)
            if cfg.is_attention(l):
                y = gated_attention_layer(cfg, W, l, h, self.caches[l], self.pos, self.cos, self.sin)
            else:
                y, self.states[l] = gated_deltanet_layer(cfg, W, l, h, self.states[l], decode)
            x = x + y
            x = x + mlp(W, l, rmsnorm_1p(x, W[p + "post_attention_layernorm"], cfg.eps))
            if l == self.steer_layer and self.vecs is not None:
                x = x.contiguous()
                ops.residual_steer_add_(x, self.vecs, self.vec_rows)
            if l == collect_layer:
                collected = x.clone()
        self.pos += T
        if stop_after is not None:
            return None, collected
        hN = rmsnorm_1p(x[:, -1], W["norm"], cfg.eps)
        return hN @ W["embed"].T, collected


@torch.no_grad()
def greedy(model, prompt_ids, steps):
    """Prefill prompt_ids [B, T], then `steps` greedy tokens (argmax, lowest index on ties, as torch.argmax and the
    WGSL argmax of engine/kernels.js:261-284). Returns (tokens [B, steps], top-2 margins [B, steps]) on the CPU."""
    logits, _ = model.forward(prompt_ids)
    toks, margins = [], []
    for _ in range(steps):
        top2 = logits.topk(2, dim=-1)
        nxt = logits.argmax(dim=-1)
        toks.append(nxt)
        margins.append(top2.values[:, 0] - top2.values[:, 1])
        logits, _ = model.forward(nxt[:, None])
    return torch.stack(toks, 1).cpu(), torch.stack(margins, 1).cpu()


def median_resid_norm(resid_row):
    """Median over tokens 1..T-1 of |x_t| (engine/analysis.js:64-74: sorted, element len >> 1)."""
    n = resid_row[1:].float().norm(dim=-1).sort().values
    return float(n[n.shape[0] >> 1])


@torch.no_grad()
def steered_greedy(model, prompt_ids, steps, steer_layer=12, dose=0.8, seed=0):
    """The three-row steering protocol: a randn(H) vector (seed `seed`) scaled to `dose` x the median residual norm
    after `steer_layer` of the unsteered prompt (tokens 1..T-1), added on row 0, absent on row 1, negated on row 2,
    at every position of the prefill and of each greedy step (engine/analysis.js:117-145 with vec rows
    [+v, none, -v] as tests/engine.html:84 sets them). Returns (tokens, margins, vector)."""
    cfg = model.cfg
    model.reset()
    model.vecs = None
    _, resid = model.forward(prompt_ids[:1], stop_after=steer_layer, collect_layer=steer_layer)
    med = median_resid_norm(resid[0])
    v = torch.randn(cfg.hidden, generator=torch.Generator().manual_seed(seed))
    v = v / v.norm() * (dose * med)
    model.set_vectors(torch.stack([v, -v]), [0, -1, 1])
    model.reset()
    toks, margins = greedy(model, prompt_ids, steps)
    return toks, margins, v
