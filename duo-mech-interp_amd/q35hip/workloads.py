"""Seeded synthetic inputs for the hot-path workloads (generated on the host in fp32, then cast / moved).

  gdn_decode:      batch 1, 16 heads, d_k = d_v = 128, 64 sequential tokens, fp32 state from 0.
  gdn_prefill:     B = 1, T = 4096, 16 heads, d_k = d_v = 128, bf16 q/k/v, chunk 64, fp32 state from 0.
  attn_prefill:    B = 1, T = 4096, causal, 8 query / 2 kv heads, head dim 256, RoPE theta 1e7 on dims 0..63,
                   gate [T, 8 * 256].
  attn_decode:     B in {3, 32}, context 8192, same heads, bf16 KV cache, one query per row, split-K.
  hybrid stack:    Qwen3.5-0.8B shape (Q35Config), seeded random weights (init_weights), every linear and the
                   tied embedding int8 with one scale per group of 128 inputs, as the engine quantizes them.
q and k are L2-normalised per head, beta = sigmoid(randn), g = -softplus(randn) (log decay, alpha = exp(g)).
"""
from dataclasses import dataclass

import torch
import torch.nn.functional as F


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def gdn_inputs(B=1, T=64, H=16, D=128, seed=0, dtype=torch.float32, normalize=True, Hk=None):
    gen = _gen(seed)
    Hk = H if Hk is None else Hk
    q = torch.randn(B, T, Hk, D, generator=gen)
    k = torch.randn(B, T, Hk, D, generator=gen)
    v = torch.randn(B, T, H, D, generator=gen)
    if normalize:
        q = F.normalize(q, dim=-1)
        k = F.normalize(k, dim=-1)
    beta = torch.sigmoid(torch.randn(B, T, H, generator=gen))
    g = -F.softplus(torch.randn(B, T, H, generator=gen))
    return dict(q=q.to(dtype), k=k.to(dtype), v=v.to(dtype), g=g, beta=beta)


def attn_prefill_inputs(B=1, T=4096, Hq=8, Hkv=2, D=256, seed=0):
    gen = _gen(seed)
    q = torch.randn(B, T, Hq, D, generator=gen).to(torch.bfloat16)
    k = torch.randn(B, T, Hkv, D, generator=gen).to(torch.bfloat16)
    v = torch.randn(B, T, Hkv, D, generator=gen).to(torch.bfloat16)
    gate = torch.randn(B, T, Hq * D, generator=gen).to(torch.bfloat16)
    return dict(q=q, k=k, v=v, gate=gate)


def attn_decode_inputs(B=3, N=8192, Hq=8, Hkv=2, D=256, seed=0, max_len=None, lens=None):
    gen = _gen(seed)
    max_len = N if max_len is None else max_len
    q = torch.randn(B, Hq, D, generator=gen).to(torch.bfloat16)
    k_cache = torch.randn(B, Hkv, max_len, D, generator=gen).to(torch.bfloat16)
    v_cache = torch.randn(B, Hkv, max_len, D, generator=gen).to(torch.bfloat16)
    gate = torch.randn(B, Hq * D, generator=gen).to(torch.bfloat16)
    cache_len = torch.full((B,), N, dtype=torch.int32) if lens is None else torch.as_tensor(lens, dtype=torch.int32)
    return dict(q=q, k_cache=k_cache, v_cache=v_cache, gate=gate, cache_len=cache_len)


def rope_tables(n_pos, head_dim=256, partial_rotary_factor=0.25, theta=1e7):
    """cos/sin tables [n_pos, rot/2] fp32, angle = pos * inv_freq with inv_freq = 1 / theta^(2j/rot) in fp32
    (the default RoPE of the Qwen3.5 text model)."""
    rot = int(head_dim * partial_rotary_factor)
    inv_freq = 1.0 / (theta ** (torch.arange(0, rot, 2, dtype=torch.int64).to(dtype=torch.float) / rot))
    ang = torch.arange(n_pos, dtype=torch.float32)[:, None] * inv_freq[None, :]
    return ang.cos().contiguous(), ang.sin().contiguous()


def to_device(d, device):
    return {k: (v.to(device) if torch.is_tensor(v) else v) for k, v in d.items()}


@dataclass
class Q35Config:
    vocab: int = 151936
    hidden: int = 1024
    inter: int = 3584
    layers: int = 24
    n_heads: int = 8
    n_kv: int = 2
    head_dim: int = 256
    lin_k_heads: int = 16
    lin_v_heads: int = 16
    lin_dk: int = 128
    lin_dv: int = 128
    conv_k: int = 4
    rope_theta: float = 1e7
    partial_rotary: float = 0.25
    eps: float = 1e-6
    full_attention_interval: int = 4
    init_std: float = 0.02
    layer_types: tuple = None  # per layer "linear_attention" / "full_attention" (a checkpoint's config); None: interval
    tie_embeddings: bool = True

    def is_attention(self, layer):
        """The checkpoint's layer_types when given, else the pattern of HFcfg:113-115: every
        full_attention_interval-th layer is full attention."""
        if self.layer_types is not None:
            return self.layer_types[layer] == "full_attention"
        return (layer + 1) % self.full_attention_interval == 0

    @property
    def conv_dim(self):
        return 2 * self.lin_k_heads * self.lin_dk + self.lin_v_heads * self.lin_dv

    @property
    def rot(self):
        return int(self.head_dim * self.partial_rotary)


def quantize_rows_int8(w):
    """Per-output-channel symmetric int8: q = round(w / s), s = max|w_row| / 127 (rows = output channels)."""
    s = w.abs().amax(dim=1, keepdim=True).clamp_min(1e-12) / 127.0
    q = torch.round(w / s).clamp(-127, 127).to(torch.int8)
    return q, s.squeeze(1).float()


QG = 128  # inputs per quantization group (engine/kernels.js:5)


def quantize_groups_int8(w, group=QG):
    """The engine's q8 format (engine/kernels.js:15-47 `quantize`): symmetric int8 with one fp32 scale per group of
    `group` consecutive inputs of a row, s = max|w_group| / 127 (1 for an all-zero group), q = round(w / s) (round
    half to even, as WGSL round and torch.round). w [N, K], K a multiple of group -> (q [N, K] int8, s [N, K / group])."""
    N, K = w.shape
    if K % group:
        raise ValueError(f"{K} inputs are not a multiple of the quantization group {group}")
    wg = w.float().reshape(N, K // group, group)
    m = wg.abs().amax(dim=2)
    s = torch.where(m == 0, torch.ones_like(m), m / 127.0)
    q = torch.round(wg / s[:, :, None]).clamp(-127, 127).to(torch.int8).reshape(N, K)
    return q, s.float()


def quantize_int8(w, group=QG):
    """int8 weights of w: per group of `group` inputs (the engine's format), or per output row when group is 0."""
    return quantize_groups_int8(w, group) if group else quantize_rows_int8(w)


def dequantize_int8(q, s):
    """fp32 values of int8 q [N, K] with scales s [N] (per row) or [N, K / g] (per group of g inputs)."""
    if s.dim() == 1:
        return q.float() * s.float()[:, None]
    N, K = q.shape
    return (q.float().reshape(N, s.shape[1], -1) * s.float()[:, :, None]).reshape(N, K)


def init_weights(cfg: Q35Config, seed=0, int8_all=True, group=QG, mlp_group=None):
    """Deterministic random init (seeded): normal(0, init_std) for every linear, the conv and the tied embedding;
    decoder / q / k RMSNorm weights 0 (gain 1 + w = 1) and the gated norm weight 1 (HF:171, HF:813-820);
    dt_bias = 1; A_log = log U(0, 16).

    Every linear layer and the tied embedding are int8 with fp32 scales, as the engine quantizes the checkpoint on
    load (engine/model.js:3-5, :70-100): one scale per group of `group` inputs (the engine's 128), or per output row
    with group 0. The MLP weights take `mlp_group` instead when it is given (0: int8 per output channel, the MLP
    format the config-5 workload states, with the other linears in the engine's format). MLP weights are stored as
    "<name>.q" / "<name>.s" only; the
    other linears and the embedding (int8_all) keep "<name>.q" / "<name>.s" beside "<name>" = the dequantised fp32
    values, so a consumer that reads "<name>" (the CPU oracle, torch GEMMs) computes with exactly the numbers the int8
    decode GEMVs use."""
    g = torch.Generator().manual_seed(seed)
    std = cfg.init_std

    def lin(o, i):
        return torch.randn(o, i, generator=g) * std

    def put(W, key, w):
        if int8_all:
            q, s = quantize_int8(w, group)
            W[key + ".q"], W[key + ".s"] = q, s
            w = dequantize_int8(q, s)
        W[key] = w

    H = cfg.hidden
    W = {"norm": torch.zeros(H)}
    put(W, "embed", torch.randn(cfg.vocab, H, generator=g) * std)
    for l in range(cfg.layers):
        p = f"layers.{l}."
        W[p + "input_layernorm"] = torch.zeros(H)
        W[p + "post_attention_layernorm"] = torch.zeros(H)
        if cfg.is_attention(l):
            put(W, p + "q_proj", lin(cfg.n_heads * cfg.head_dim * 2, H))
            put(W, p + "k_proj", lin(cfg.n_kv * cfg.head_dim, H))
            put(W, p + "v_proj", lin(cfg.n_kv * cfg.head_dim, H))
            put(W, p + "o_proj", lin(H, cfg.n_heads * cfg.head_dim))
            W[p + "q_norm"] = torch.zeros(cfg.head_dim)
            W[p + "k_norm"] = torch.zeros(cfg.head_dim)
        else:
            vd = cfg.lin_v_heads * cfg.lin_dv
            put(W, p + "in_proj_qkv", lin(cfg.conv_dim, H))
            put(W, p + "in_proj_z", lin(vd, H))
            put(W, p + "in_proj_b", lin(cfg.lin_v_heads, H))
            put(W, p + "in_proj_a", lin(cfg.lin_v_heads, H))
            W[p + "conv1d"] = torch.randn(cfg.conv_dim, cfg.conv_k, generator=g) * std
            W[p + "dt_bias"] = torch.ones(cfg.lin_v_heads)
            W[p + "A_log"] = torch.empty(cfg.lin_v_heads).uniform_(0, 16, generator=g).log()
            W[p + "norm"] = torch.ones(cfg.lin_dv)
            put(W, p + "out_proj", lin(H, vd))
        for name, (o, i) in (("gate_proj", (cfg.inter, H)), ("up_proj", (cfg.inter, H)), ("down_proj", (H, cfg.inter))):
            q, s = quantize_int8(lin(o, i), group if mlp_group is None else mlp_group)
            W[p + name + ".q"] = q
            W[p + name + ".s"] = s
    return W
