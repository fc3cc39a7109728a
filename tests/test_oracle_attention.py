"""Pins the gated attention oracle: a library routine (scaled_dot_product_attention), a brute-force loop, RoPE closed
forms, decode = last prefill row. CPU only."""
import math

import pytest
import torch
import torch.nn.functional as F

import oracle
from q35hip import workloads


def test_prefill_matches_sdpa_and_gate():
    inp = workloads.attn_prefill_inputs(B=2, T=33, Hq=8, Hkv=2, seed=1)
    cos, sin = workloads.rope_tables(40)
    got = oracle.gated_attention(inp["q"], inp["k"], inp["v"], inp["gate"], cos, sin, pos0=3, dtype=torch.float64)
    q = oracle.apply_partial_rope(inp["q"].double(), cos[3:36].double(), sin[3:36].double())
    k = oracle.apply_partial_rope(inp["k"].double(), cos[3:36].double(), sin[3:36].double())
    ref = F.scaled_dot_product_attention(q.transpose(1, 2), k.transpose(1, 2), inp["v"].double().transpose(1, 2),
                                         is_causal=True, enable_gqa=True)
    ref = ref.transpose(1, 2).reshape(2, 33, -1) * torch.sigmoid(inp["gate"].double())
    assert oracle.rel_err(got, ref) < 1e-12


def test_brute_force_single_query():
    inp = workloads.attn_prefill_inputs(B=1, T=6, Hq=4, Hkv=2, seed=2)
    got = oracle.gated_attention(inp["q"], inp["k"], inp["v"], inp["gate"], None, None, dtype=torch.float64)
    q, k, v, gate = [inp[n].double() for n in ("q", "k", "v", "gate")]
    t, h = 4, 3
    kv = h // 2
    s = [float((q[0, t, h] * k[0, j, kv]).sum()) / 16.0 for j in range(t + 1)]
    m = max(s)
    w = [math.exp(x - m) for x in s]
    o = sum(w[j] * v[0, j, kv] for j in range(t + 1)) / sum(w)
    want = o * torch.sigmoid(gate[0, t, h * 256:(h + 1) * 256])
    assert torch.allclose(got[0, t, h * 256:(h + 1) * 256], want, atol=1e-12)


def test_rope_closed_forms():
    cos, sin = workloads.rope_tables(300)
    x = torch.randn(1, 300, 1, 256, dtype=torch.float64)
    y = oracle.apply_partial_rope(x, cos.double(), sin.double())
    # position 0 is the identity; dims >= 64 pass through; each (i, i + 32) pair keeps its norm
    assert torch.allclose(y[:, 0], x[:, 0])
    assert torch.equal(y[..., 64:], x[..., 64:])
    n0 = x[..., :32] ** 2 + x[..., 32:64] ** 2
    n1 = y[..., :32] ** 2 + y[..., 32:64] ** 2
    assert torch.allclose(n0, n1)
    # hand-computed pair: dims (0, 32) rotate by angle pos * inv_freq_0 = pos
    p = 7
    a = x[0, p, 0, 0] * math.cos(p) - x[0, p, 0, 32] * math.sin(p)
    assert abs(float(y[0, p, 0, 0] - a)) < 1e-5
    # relative position: q_m . k_n depends on m - n only
    q = torch.randn(256, dtype=torch.float64)
    k = torch.randn(256, dtype=torch.float64)
    def rot(v, pos):
        return oracle.apply_partial_rope(v[None, None, None], cos[pos:pos + 1].double(), sin[pos:pos + 1].double())[0, 0, 0]
    d1 = float((rot(q, 100) * rot(k, 90)).sum())
    d2 = float((rot(q, 210) * rot(k, 200)).sum())
    assert abs(d1 - d2) < 1e-4 * (1 + abs(d1))


def test_inv_freq_matches_hf_formula():
    f = oracle.rope_inv_freq(256, 0.25, 1e7)
    assert f.shape == (32,) and f.dtype == torch.float32
    assert abs(float(f[1]) - 1e7 ** (-2 / 64)) < 1e-7 and float(f[0]) == 1.0


def test_decode_equals_last_prefill_row():
    T = 20
    inp = workloads.attn_prefill_inputs(B=1, T=T, Hq=8, Hkv=2, seed=5)
    cos, sin = workloads.rope_tables(T)
    full = oracle.gated_attention(inp["q"], inp["k"], inp["v"], inp["gate"], cos, sin, dtype=torch.float64)
    k_rot = oracle.apply_partial_rope(inp["k"].double(), cos.double(), sin.double())
    dec = oracle.gated_attention_decode(inp["q"][:, T - 1], k_rot.transpose(1, 2), inp["v"].transpose(1, 2),
                                        inp["gate"][:, T - 1], [T], cos, sin, dtype=torch.float64)
    assert oracle.rel_err(dec, full[:, T - 1]) < 1e-6


def _rotated_cache(k, v, cos, sin, max_len):
    """Caches [B, Hkv, max_len, D] holding k (rotated at positions 0..T-1) and v, the rest random."""
    B, T, Hkv, D = k.shape
    kr = oracle.apply_partial_rope(k.double(), cos[:T].double(), sin[:T].double())
    g = torch.Generator().manual_seed(7)
    kc = torch.randn(B, Hkv, max_len, D, generator=g, dtype=torch.float64)
    vc = torch.randn(B, Hkv, max_len, D, generator=g, dtype=torch.float64)
    kc[:, :, :T] = kr.transpose(1, 2)
    vc[:, :, :T] = v.double().transpose(1, 2)
    return kc, vc


def test_cached_form_equals_self_form_decode_and_split_prompt():
    """The cached form reduces to the self form at position 0 (cache = the call's rotated keys), to decode for
    T = 1, and a prompt attended in two calls (positions 0..P-1, then P..T-1 over the cache) equals one call."""
    inp = workloads.attn_prefill_inputs(B=2, T=50, Hq=8, Hkv=2, seed=4)
    cos, sin = workloads.rope_tables(64)
    q, k, v, gate = inp["q"], inp["k"], inp["v"], inp["gate"]
    kc, vc = _rotated_cache(k, v, cos, sin, 64)
    whole = oracle.gated_attention(q, k, v, gate, cos, sin, dtype=torch.float64)
    z = torch.zeros(2, dtype=torch.int64)
    got = oracle.gated_attention_cached(q, kc, vc, gate, z, cos, sin, dtype=torch.float64)
    assert oracle.rel_err(got, whole) < 1e-12
    P = 37
    tail = oracle.gated_attention_cached(q[:, P:], kc, vc, gate[:, P:], z + P, cos, sin, dtype=torch.float64)
    assert oracle.rel_err(tail, whole[:, P:]) < 1e-12
    dec = oracle.gated_attention_decode(q[:, P], kc, vc, gate[:, P], z + P + 1, cos, sin, dtype=torch.float64)
    one = oracle.gated_attention_cached(q[:, P:P + 1], kc, vc, gate[:, P:P + 1], z + P, cos, sin,
                                        dtype=torch.float64)
    assert oracle.rel_err(one[:, 0], dec) < 1e-12
    # a planted off-by-one in the key range must be caught by the split-prompt identity
    bad = oracle.gated_attention_cached(q[:, P:], kc, vc, gate[:, P:], z + P + 1, cos, sin, dtype=torch.float64)
    assert oracle.rel_err(bad, whole[:, P:]) > 1e-3


def test_cached_form_rows_at_different_positions():
    """Each row of a cached call depends only on its own position and cache: rows computed together equal rows
    computed alone."""
    inp = workloads.attn_prefill_inputs(B=3, T=20, Hq=4, Hkv=1, seed=5)
    cos, sin = workloads.rope_tables(128)
    g = torch.Generator().manual_seed(8)
    kc = torch.randn(3, 1, 128, 256, generator=g, dtype=torch.float64)
    vc = torch.randn(3, 1, 128, 256, generator=g, dtype=torch.float64)
    pos = torch.tensor([0, 13, 100])
    both = oracle.gated_attention_cached(inp["q"], kc, vc, inp["gate"], pos, cos, sin, dtype=torch.float64)
    for b in range(3):
        one = oracle.gated_attention_cached(inp["q"][b:b + 1], kc[b:b + 1], vc[b:b + 1], inp["gate"][b:b + 1],
                                            pos[b:b + 1], cos, sin, dtype=torch.float64)
        assert torch.equal(one[0], both[b])
