"""Gated attention parity on the GPU: HIP prefill / decode kernels against the CPU oracle in fp32 on the same
bf16-rounded inputs (relative error <= 2e-2, the bf16-activation tolerance)."""
import pytest
import torch

import oracle
import q35hip
from q35hip import workloads
from gpu_util import announce, device

pytestmark = pytest.mark.gpu
TOL = 2e-2


def _tables(n):
    return workloads.rope_tables(n)


# T >= 449 (at least 8 key tiles in the last query block) may run the long query blocks as two key-split halves that
# are merged in a third kernel, when the launcher's dispatch estimate finds that faster than whole blocks on 256
# CUs. T 1000 and 777 (GQA 4 and 1) split and fit the device as paired items (the second half of a long block, then
# a short whole block, in one block; 777 leaves whole blocks unpaired); T 5120 splits into more items than CUs and
# runs them independently, longest first; B 2 T 600 GQA 8 (two head groups per kv head), B 4 T 1000 GQA 1 and B 5
# T 1000 GQA 2 run whole blocks longest first (their longest block is short against a CU's share).
@pytest.mark.parametrize("B,T,Hq,Hkv,pos0", [(1, 1, 8, 2, 0), (2, 100, 8, 2, 0), (1, 257, 8, 2, 5),
                                             (1, 96, 4, 4, 0), (1, 70, 8, 1, 3), (1, 64, 16, 2, 0),
                                             (1, 1000, 8, 2, 3), (2, 600, 16, 2, 0), (1, 777, 4, 4, 0),
                                             (4, 1000, 8, 8, 0), (5, 1000, 4, 2, 1), (1, 5120, 8, 2, 0)])
def test_prefill_small(B, T, Hq, Hkv, pos0):
    dev = device()
    inp = workloads.attn_prefill_inputs(B=B, T=T, Hq=Hq, Hkv=Hkv, seed=T)
    cos, sin = _tables(pos0 + T)
    ref = oracle.gated_attention(inp["q"], inp["k"], inp["v"], inp["gate"], cos, sin, pos0=pos0)
    d = workloads.to_device(inp, dev)
    announce(f"attn prefill B{B} T{T} Hq{Hq} Hkv{Hkv} pos0 {pos0}")
    out = q35hip.gated_attention_prefill(d["q"], d["k"], d["v"], d["gate"], cos.to(dev), sin.to(dev), pos0=pos0)
    assert oracle.rel_err(out.float().cpu(), ref) <= TOL


def test_prefill_full_size():
    """B = 1, T = 4096, causal, 8 q / 2 kv heads, head dim 256, RoPE theta 1e7 on dims 0..63, sigmoid gate."""
    dev = device()
    inp = workloads.attn_prefill_inputs(B=1, T=4096, seed=0)
    cos, sin = _tables(4096)
    ref = oracle.gated_attention(inp["q"], inp["k"], inp["v"], inp["gate"], cos, sin)
    d = workloads.to_device(inp, dev)
    announce("attn prefill T4096 (full size)")
    out = q35hip.gated_attention_prefill(d["q"], d["k"], d["v"], d["gate"], cos.to(dev), sin.to(dev))
    e = oracle.rel_err(out.float().cpu(), ref)
    print(f"attn prefill T4096 rel err {e:.3e}")
    assert e <= TOL
    # the split blocks' merge does not depend on which half finishes last: repeated calls agree bitwise
    for _ in range(3):
        again = q35hip.gated_attention_prefill(d["q"], d["k"], d["v"], d["gate"], cos.to(dev), sin.to(dev))
        assert torch.equal(again, out)


def test_prefill_long_sequence():
    """T = 8192 (256 whole query blocks per kv head, longest first: the longest block's 128 tiles are about a CU's
    share, so nothing is split) against the fp32 oracle."""
    dev = device()
    inp = workloads.attn_prefill_inputs(B=1, T=8192, seed=9)
    cos, sin = _tables(8192)
    ref = oracle.gated_attention(inp["q"], inp["k"], inp["v"], inp["gate"], cos, sin)
    d = workloads.to_device(inp, dev)
    announce("attn prefill T8192")
    out = q35hip.gated_attention_prefill(d["q"], d["k"], d["v"], d["gate"], cos.to(dev), sin.to(dev))
    e = oracle.rel_err(out.float().cpu(), ref)
    print(f"attn prefill T8192 rel err {e:.3e}")
    assert e <= TOL


def _score_regime(q, k, regime, key_axis):
    """Reshape the scores so that the softmax's running max moves: `rising` adds 16 u to every query and
    60 (t / T) u to key t (u the unit vector on dims 192..255, outside the rotary dims), a score drift of 60 / sqrt(256)
    x 16 = 60 nats over the keys, so later tiles keep beating the running max by more than the prefill kernel's
    2^8 rescale threshold; `sharp` multiplies the queries by 8 (scores with a standard deviation of about 8: near
    one-hot rows whose maxima jump between tiles)."""
    if regime == "sharp":
        return (q.float() * 8).to(torch.bfloat16), k
    D = q.shape[-1]
    u = torch.zeros(D)
    u[192:] = 64 ** -0.5
    n = k.shape[key_axis]
    shape = [1] * k.dim()
    shape[key_axis] = n
    ramp = (torch.arange(n, dtype=torch.float32) / n).view(shape)
    return (q.float() + 16 * u).to(torch.bfloat16), (k.float() + 60 * ramp * u).to(torch.bfloat16)


@pytest.mark.parametrize("regime,T", [("rising", 1000), ("sharp", 1000), ("rising", 4096)])
def test_prefill_running_max_moves(regime, T):
    """Prefill with scores whose running max moves tile after tile (the rescale of O and l outside the kernel's inner
    loop, and split halves whose maxima differ by tens of nats in the merge), against the fp32 oracle."""
    dev = device()
    inp = workloads.attn_prefill_inputs(B=1, T=T, seed=40 + T)
    q, k = _score_regime(inp["q"], inp["k"], regime, key_axis=1)
    inp = dict(inp, q=q, k=k)
    cos, sin = _tables(T)
    ref = oracle.gated_attention(inp["q"], inp["k"], inp["v"], inp["gate"], cos, sin)
    d = workloads.to_device(inp, dev)
    announce(f"attn prefill T{T} scores {regime}")
    out = q35hip.gated_attention_prefill(d["q"], d["k"], d["v"], d["gate"], cos.to(dev), sin.to(dev))
    e = oracle.rel_err(out.float().cpu(), ref)
    print(f"attn prefill T{T} {regime}: rel err {e:.3e}")
    assert torch.isfinite(out.float()).all()
    assert e <= TOL


@pytest.mark.parametrize("regime", ["rising", "sharp"])
def test_decode_running_max_moves(regime):
    """Decode over 8192 cached keys with rising or sharp scores: the splits' partial maxima differ by tens of nats,
    so the merge's weights 2^(m_s - m) span a wide range; rows of 8192, 5000 and 1 keys."""
    dev = device()
    inp = workloads.attn_decode_inputs(B=3, N=8192, seed=41, lens=[8192, 5000, 1])
    q, kc = _score_regime(inp["q"], inp["k_cache"], regime, key_axis=2)
    inp = dict(inp, q=q, k_cache=kc)
    cos, sin = _tables(8192)
    ref = oracle.gated_attention_decode(inp["q"], inp["k_cache"], inp["v_cache"], inp["gate"], inp["cache_len"],
                                        cos, sin)
    d = workloads.to_device(inp, dev)
    announce(f"attn decode B3 N8192 scores {regime}")
    out = q35hip.gated_attention_decode(d["q"], d["k_cache"], d["v_cache"], d["gate"], d["cache_len"],
                                        cos.to(dev), sin.to(dev))
    e = oracle.rel_err(out.float().cpu(), ref)
    print(f"attn decode {regime}: rel err {e:.3e}")
    assert torch.isfinite(out.float()).all()
    assert e <= TOL


@pytest.mark.parametrize("B", [3, 32])
def test_decode_full_size(B):
    """Batch 3 and 32, context 8192, 8 q / 2 kv heads, head dim 256, bf16 KV cache, split-K."""
    dev = device()
    inp = workloads.attn_decode_inputs(B=B, N=8192, seed=B)
    cos, sin = _tables(8192)
    ref = oracle.gated_attention_decode(inp["q"], inp["k_cache"], inp["v_cache"], inp["gate"], inp["cache_len"],
                                        cos, sin)
    d = workloads.to_device(inp, dev)
    announce(f"attn decode B{B} N8192")
    out = q35hip.gated_attention_decode(d["q"], d["k_cache"], d["v_cache"], d["gate"], d["cache_len"],
                                        cos.to(dev), sin.to(dev))
    e = oracle.rel_err(out.float().cpu(), ref)
    print(f"attn decode B{B} rel err {e:.3e}")
    assert e <= TOL


@pytest.mark.parametrize("splits", [1, 2, 7, 0, 64])
def test_decode_ragged_lengths_and_split_invariance(splits):
    dev = device()
    lens = [1, 17, 300, 1000]
    inp = workloads.attn_decode_inputs(B=4, N=1000, max_len=1024, seed=4, lens=lens)
    cos, sin = _tables(1024)
    ref = oracle.gated_attention_decode(inp["q"], inp["k_cache"], inp["v_cache"], inp["gate"], inp["cache_len"],
                                        cos, sin)
    d = workloads.to_device(inp, dev)
    announce(f"attn decode ragged splits {splits}")
    out = q35hip.gated_attention_decode(d["q"], d["k_cache"], d["v_cache"], d["gate"], d["cache_len"],
                                        cos.to(dev), sin.to(dev), splits=splits)
    assert oracle.rel_err(out.float().cpu(), ref) <= TOL


def test_decode_matches_last_prefill_row():
    """Decode of token T-1 over the rotated K cache of a prefill equals the prefill's last output row."""
    dev = device()
    T = 300
    inp = workloads.attn_prefill_inputs(B=1, T=T, seed=12)
    cos, sin = _tables(T)
    d = workloads.to_device(inp, dev)
    announce("attn decode vs prefill last row")
    full = q35hip.gated_attention_prefill(d["q"], d["k"], d["v"], d["gate"], cos.to(dev), sin.to(dev))
    k_rot = oracle.apply_partial_rope(inp["k"].float(), cos, sin).to(torch.bfloat16)  # [1, T, Hkv, D]
    k_cache = k_rot.transpose(1, 2).contiguous().to(dev)
    v_cache = inp["v"].transpose(1, 2).contiguous().to(dev)
    q_last = d["q"][:, T - 1].contiguous()
    gate_last = d["gate"][:, T - 1].contiguous()
    cl = torch.tensor([T], dtype=torch.int32, device=dev)
    dec = q35hip.gated_attention_decode(q_last, k_cache, v_cache, gate_last, cl, cos.to(dev), sin.to(dev))
    assert oracle.rel_err(dec.float().cpu(), full[:, T - 1].float().cpu()) <= TOL


def test_decode_fp32_output_is_the_unrounded_bf16_output():
    """out_dtype=float32 writes the merge kernel's fp32 result (the stack's o_proj input); rounded to bf16 it is the
    bf16 output bit for bit, and it matches the oracle within the fp32 arithmetic's error."""
    dev = device()
    inp = workloads.attn_decode_inputs(B=3, N=777, max_len=1024, seed=8, lens=[777, 1, 300])
    cos, sin = _tables(1024)
    ref = oracle.gated_attention_decode(inp["q"], inp["k_cache"], inp["v_cache"], inp["gate"], inp["cache_len"],
                                        cos, sin)
    d = workloads.to_device(inp, dev)
    announce("attn decode fp32 output")
    args = (d["q"], d["k_cache"], d["v_cache"], d["gate"], d["cache_len"], cos.to(dev), sin.to(dev))
    o16 = q35hip.gated_attention_decode(*args)
    o32 = q35hip.gated_attention_decode(*args, out_dtype=torch.float32)
    assert o32.dtype == torch.float32 and o16.dtype == torch.bfloat16
    assert torch.equal(o32.to(torch.bfloat16).cpu(), o16.cpu())
    assert oracle.rel_err(o32.cpu(), ref) <= TOL


# Multi-token calls over a KV cache at per-row positions: token t of row b attends to cache keys 0 .. pos[b] + t.
# Cases: rows at different positions, one token, a query length past 256 with the keys filling the cache exactly,
# GQA 8 with a row at position 0, two head groups per kv head.
@pytest.mark.parametrize("B,T,Hq,Hkv,max_len,pos", [(3, 100, 8, 2, 448, [0, 37, 300]), (2, 1, 8, 2, 256, [5, 200]),
                                                     (1, 257, 4, 4, 640, [383]), (2, 64, 8, 1, 192, [128, 0]),
                                                     (1, 130, 16, 2, 320, [64])])
def test_prefill_over_cache(B, T, Hq, Hkv, max_len, pos):
    dev = device()
    inp = workloads.attn_prefill_inputs(B=B, T=T, Hq=Hq, Hkv=Hkv, seed=T + max_len)
    g = torch.Generator().manual_seed(max_len)
    kc = torch.randn(B, Hkv, max_len, 256, generator=g).to(torch.bfloat16)
    vc = torch.randn(B, Hkv, max_len, 256, generator=g).to(torch.bfloat16)
    cos, sin = _tables(max_len)
    pos_t = torch.tensor(pos, dtype=torch.int32)
    ref = oracle.gated_attention_cached(inp["q"], kc, vc, inp["gate"], pos_t, cos, sin)
    announce(f"attn prefill over cache B{B} T{T} Hq{Hq} Hkv{Hkv} max_len {max_len} pos {pos}")
    out = q35hip.ops.gated_attention_prefill_cached(inp["q"].to(dev), kc.to(dev), vc.to(dev), inp["gate"].to(dev),
                                                    pos_t.to(dev), cos.to(dev), sin.to(dev))
    e = oracle.rel_err(out.float().cpu(), ref)
    print(f"cached prefill rel err {e:.3e}")
    assert e <= TOL


def test_prefill_over_cache_equals_own_keys_at_position_zero():
    """At position 0 with the cache holding the call's rotated keys, the cached path gives the own-keys path's
    result to bf16 rounding. Not bitwise: the cache's keys are rotated on the host here (the own-keys path rotates
    them on the GPU, each rounded to bf16), and the own-keys path splits long query blocks into two key ranges merged
    afterwards (another summation order); both differences are at bf16 rounding, well inside the bound."""
    dev = device()
    B, T, max_len = 2, 200, 256
    inp = workloads.to_device(workloads.attn_prefill_inputs(B=B, T=T, seed=9), dev)
    cos, sin = [t.to(dev) for t in _tables(max_len)]
    kr = oracle.apply_partial_rope(inp["k"].float().cpu(), cos[:T].cpu(), sin[:T].cpu()).to(torch.bfloat16)
    kc = torch.zeros(B, 2, max_len, 256, dtype=torch.bfloat16, device=dev)
    vc = torch.zeros_like(kc)
    kc[:, :, :T] = kr.transpose(1, 2).to(dev)
    vc[:, :, :T] = inp["v"].transpose(1, 2)
    announce("attn prefill over cache at position 0 vs own keys")
    own = q35hip.gated_attention_prefill(inp["q"], inp["k"], inp["v"], inp["gate"], cos, sin)
    cached = q35hip.ops.gated_attention_prefill_cached(inp["q"], kc, vc, inp["gate"],
                                                       torch.zeros(B, dtype=torch.int32, device=dev), cos, sin)
    e = oracle.rel_err(cached.float().cpu(), own.float().cpu())
    print(f"cached vs own keys at position 0: rel err {e:.2e}")
    assert e <= 1e-2
