"""Seeded synthetic inputs for the hot-path workloads (generated on the host in fp32, then cast / moved).

  gdn_decode:      batch 1, 16 heads, d_k = d_v = 128, 64 sequential tokens, fp32 state from 0.
  gdn_prefill:     B = 1, T = 4096, 16 heads, d_k = d_v = 128, bf16 q/k/v, chunk 64, fp32 state from 0.
  attn_prefill:    B = 1, T = 4096, causal, 8 query / 2 kv heads, head dim 256, RoPE theta 1e7 on dims 0..63,
                   gate [T, 8 * 256].
  attn_decode:     B in {3, 32}, context 8192, same heads, bf16 KV cache, one query per row, split-K.
q and k are L2-normalised per head, beta = sigmoid(randn), g = -softplus(randn) (log decay, alpha = exp(g)).
"""
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
