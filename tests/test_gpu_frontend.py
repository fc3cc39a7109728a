"""Layer front ends on the GPU (conv + gates, gated RMSNorm, attention prep) against the CPU oracle.

Tolerances (relative error, tests/engine.mjs:17): fp32 outputs <= 1e-5 (the kernels compute in fp32; only the
summation order differs); bf16 outputs <= 4e-3 (one rounding to bf16, 2^-9 relative, on top of fp32 arithmetic).
"""
import pytest
import torch

import oracle
import q35hip
from oracle import frontend as of
from oracle.attention import rope_inv_freq, rope_tables
from q35hip import ops
from gpu_util import announce, device

pytestmark = pytest.mark.gpu

TOL_F32 = 1e-5
TOL_BF16 = 4e-3


def _gdn_case(B, T, seed, Hk=16, dk=128, Hv=16, dv=128, K=4):
    g = torch.Generator().manual_seed(seed)
    C = 2 * Hk * dk + Hv * dv
    W = C + Hv * dv + 2 * Hv          # [qkv | z | b | a], the fused projection row
    y = torch.randn(B, T, W, generator=g)
    conv_w = 0.5 * torch.randn(C, K, generator=g)
    state = torch.randn(B, K - 1, C, generator=g)
    A_log = torch.log(torch.rand(Hv, generator=g) * 16)
    dt_bias = torch.ones(Hv) + 0.1 * torch.randn(Hv, generator=g)
    return y, conv_w, state, A_log, dt_bias, C, W


@pytest.mark.parametrize("T", [1, 2, 5, 37])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_gdn_conv_matches_oracle(T, dtype):
    dev = device()
    B, Hk, dk, Hv, dv = 3, 16, 128, 16, 128
    y, conv_w, state, A_log, dt_bias, C, W = _gdn_case(B, T, seed=T)
    b_off, a_off = C + Hv * dv, C + Hv * dv + Hv
    ref = of.gdn_conv(y, conv_w, state, A_log, dt_bias, Hk, dk, Hv, dv, b_off, a_off)
    announce(f"gdn_conv T{T} {dtype}")
    st = state.to(dev)
    out = ops.gdn_conv(y.to(dev), conv_w.to(dev), st, A_log.to(dev), dt_bias.to(dev), num_k_heads=Hk, head_k_dim=dk,
                       num_v_heads=Hv, head_v_dim=dv, b_off=b_off, a_off=a_off, out_dtype=dtype)
    torch.cuda.synchronize()
    tol = TOL_F32 if dtype == torch.float32 else TOL_BF16
    for got, exp in zip(out[:3], ref[:3]):
        assert got.dtype == dtype and got.is_contiguous()
        assert oracle.rel_err(got.float().cpu(), exp) <= tol
    for got, exp in zip(out[3:], ref[3:5]):
        assert oracle.rel_err(got.cpu(), exp) <= TOL_F32
    assert torch.equal(st.cpu(), ref[5])   # the state is a copy of inputs: exact


def test_gdn_conv_bias_and_split_calls():
    """Optional conv bias; a 37-token call equals 5 + 32 tokens with the state carried on the device."""
    dev = device()
    B, Hk, dk, Hv, dv = 2, 16, 128, 16, 128
    y, conv_w, state, A_log, dt_bias, C, W = _gdn_case(B, 37, seed=40)
    bias = torch.randn(C, generator=torch.Generator().manual_seed(41))
    b_off, a_off = C + Hv * dv, C + Hv * dv + Hv
    ref = of.gdn_conv(y, conv_w, state, A_log, dt_bias, Hk, dk, Hv, dv, b_off, a_off, conv_bias=bias)
    announce("gdn_conv bias + split calls")
    kw = dict(num_k_heads=Hk, head_k_dim=dk, num_v_heads=Hv, head_v_dim=dv, b_off=b_off, a_off=a_off)
    st = state.to(dev)
    yd = y.to(dev)
    args = (conv_w.to(dev), st, A_log.to(dev), dt_bias.to(dev))
    a = ops.gdn_conv(yd[:, :5].contiguous(), *args, conv_bias=bias.to(dev), **kw)
    b = ops.gdn_conv(yd[:, 5:].contiguous(), *args, conv_bias=bias.to(dev), **kw)
    torch.cuda.synchronize()
    for i in range(5):
        got = torch.cat([a[i], b[i]], dim=1).cpu()
        assert oracle.rel_err(got, ref[i]) <= TOL_F32
    assert torch.equal(st.cpu(), ref[5])


def test_gdn_conv_single_token_steps_carry_the_state():
    """Six one-token calls (the decode form, its own kernel) equal one six-token call, bias included, for both
    output dtypes; the carried state ends identical."""
    dev = device()
    B, Hk, dk, Hv, dv = 3, 16, 128, 16, 128
    y, conv_w, state, A_log, dt_bias, C, W = _gdn_case(B, 6, seed=44)
    bias = torch.randn(C, generator=torch.Generator().manual_seed(45))
    b_off, a_off = C + Hv * dv, C + Hv * dv + Hv
    ref = of.gdn_conv(y, conv_w, state, A_log, dt_bias, Hk, dk, Hv, dv, b_off, a_off, conv_bias=bias)
    kw = dict(num_k_heads=Hk, head_k_dim=dk, num_v_heads=Hv, head_v_dim=dv, b_off=b_off, a_off=a_off)
    for dtype in (torch.float32, torch.bfloat16):
        announce(f"gdn_conv one-token steps {dtype}")
        st = state.to(dev)
        yd = y.to(dev)
        outs = [ops.gdn_conv(yd[:, t:t + 1].contiguous(), conv_w.to(dev), st, A_log.to(dev), dt_bias.to(dev),
                             conv_bias=bias.to(dev), out_dtype=dtype, **kw) for t in range(6)]
        torch.cuda.synchronize()
        tol = TOL_F32 if dtype == torch.float32 else TOL_BF16
        for i in range(5):
            got = torch.cat([o[i] for o in outs], dim=1).float().cpu()
            assert oracle.rel_err(got, ref[i]) <= (tol if i < 3 else TOL_F32)
        assert torch.equal(st.cpu(), ref[5])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("with_scale", [False, True])
def test_gated_rmsnorm_matches_oracle(dtype, with_scale):
    dev = device()
    g = torch.Generator().manual_seed(50)
    B, T, Hv, dv = 3, 7, 16, 128
    o = torch.randn(B, T, Hv, dv, generator=g).to(dtype)
    y = torch.randn(B, T, 3 * Hv * dv, generator=g)            # z is a strided column range of a wider row
    z = y[..., Hv * dv:2 * Hv * dv]
    w = torch.randn(dv, generator=g)
    hs = torch.rand(Hv, generator=g) + 0.5 if with_scale else None
    ref = of.gated_rmsnorm(o, z, w, hs)
    announce(f"gated_rmsnorm {dtype} scale={with_scale}")
    yd = y.to(dev)
    out = ops.gated_rmsnorm(o.to(dev), yd[..., Hv * dv:2 * Hv * dv], w.to(dev),
                            None if hs is None else hs.to(dev))
    torch.cuda.synchronize()
    assert out.dtype == dtype and tuple(out.shape) == (B, T, Hv * dv)
    tol = TOL_F32 if dtype == torch.float32 else TOL_BF16
    assert oracle.rel_err(out.float().cpu(), ref.float()) <= tol


@pytest.mark.parametrize("T", [1, 6])
def test_attn_prep_matches_oracle_and_writes_cache_rows(T):
    dev = device()
    g = torch.Generator().manual_seed(60 + T)
    B, Hq, Hkv, D, max_len = 3, 8, 2, 256, 128
    y = torch.randn(B, T, Hq * 2 * D + 2 * Hkv * D, generator=g)
    qw, kw = 0.1 * torch.randn(D, generator=g), 0.1 * torch.randn(D, generator=g)
    cos, sin = rope_tables(max_len, rope_inv_freq(D, 0.25, 1e7))
    pos = torch.tensor([0, 10, max_len - T], dtype=torch.int32)
    q, gate, k, v, k_rot = of.attn_prep(y, qw, kw, cos, sin, pos, Hq, Hkv, D)
    announce(f"attn_prep T{T}")
    sentinel = torch.full((B, Hkv, max_len, D), 7.0, dtype=torch.bfloat16)
    kc, vc = sentinel.to(dev), sentinel.to(dev)
    out = ops.attn_prep(y.to(dev), qw.to(dev), kw.to(dev), cos.to(dev), sin.to(dev), pos.to(dev), kc, vc,
                        num_heads=Hq, num_kv_heads=Hkv)
    torch.cuda.synchronize()
    for got, exp in zip(out, (q, gate, k, v)):
        assert got.dtype == torch.bfloat16
        assert oracle.rel_err(got.float().cpu(), exp) <= TOL_BF16
    kc, vc = kc.cpu(), vc.cpu()
    written = torch.zeros(B, max_len, dtype=torch.bool)
    for b in range(B):
        p0 = int(pos[b])
        written[b, p0:p0 + T] = True
        assert oracle.rel_err(kc[b, :, p0:p0 + T].float(), k_rot[b].transpose(0, 1)) <= TOL_BF16
        assert oracle.rel_err(vc[b, :, p0:p0 + T].float(), v[b].transpose(0, 1)) <= TOL_BF16
    # every other cache row is untouched
    assert bool((kc.transpose(1, 2)[~written] == 7.0).all()) and bool((vc.transpose(1, 2)[~written] == 7.0).all())


@pytest.mark.parametrize("Hq,Hkv,splits", [(8, 2, 0), (16, 2, 0), (8, 8, 3)])
def test_attn_decode_from_projection(Hq, Hkv, splits):
    """The decode step from the fused projection output (q35_gated_attn_decode_proj: the front end inside the decode
    kernels) against the oracle's front end + decode over the cache with the token's key appended, and against the
    two-launch path (q35_attn_prep, then q35_gated_attn_decode) on the same inputs, whose caches it must leave
    bitwise equal. Rows at positions 0 (empty cache: the token attends to itself only), 1, 300 and max_len - 1; GQA
    4, 8 and 1 (with 3 splits)."""
    dev = device()
    g = torch.Generator().manual_seed(80 + Hq + Hkv)
    B, D, max_len = 4, 256, 512
    y = torch.randn(B, Hq * 2 * D + 2 * Hkv * D, generator=g)
    qw, kw = 0.1 * torch.randn(D, generator=g), 0.1 * torch.randn(D, generator=g)
    cos, sin = rope_tables(max_len, rope_inv_freq(D, 0.25, 1e7))
    pos = torch.tensor([0, 1, 300, max_len - 1], dtype=torch.int32)
    kc0 = torch.randn(B, Hkv, max_len, D, generator=g).to(torch.bfloat16)
    vc0 = torch.randn(B, Hkv, max_len, D, generator=g).to(torch.bfloat16)
    q, gate, k, v, k_rot = of.attn_prep(y[:, None], qw, kw, cos, sin, pos, Hq, Hkv, D)
    kr, vr = kc0.clone(), vc0.clone()
    for b in range(B):
        kr[b, :, int(pos[b])] = k_rot[b, 0].to(torch.bfloat16)
        vr[b, :, int(pos[b])] = v[b, 0].to(torch.bfloat16)
    ref = oracle.gated_attention_decode(q[:, 0], kr, vr, gate[:, 0], pos + 1, cos, sin)
    announce(f"attn decode from projection Hq{Hq} Hkv{Hkv} splits {splits}")
    yd, qwd, kwd, posd = y.to(dev), qw.to(dev), kw.to(dev), pos.to(dev)
    cosd, sind = cos.to(dev), sin.to(dev)
    kcb, vcb = kc0.to(dev), vc0.to(dev)
    out = ops.gated_attention_decode_proj(yd, qwd, kwd, kcb, vcb, posd, cosd, sind, num_heads=Hq, splits=splits)
    kca, vca = kc0.to(dev), vc0.to(dev)
    qa, ga, _, _ = ops.attn_prep(yd[:, None].contiguous(), qwd, kwd, cosd, sind, posd, kca, vca, num_heads=Hq,
                                 num_kv_heads=Hkv)
    two = q35hip.gated_attention_decode(qa[:, 0].contiguous(), kca, vca, ga[:, 0].contiguous(), posd + 1, cosd, sind,
                                        splits=splits)
    torch.cuda.synchronize()
    assert torch.equal(kcb.cpu(), kca.cpu()) and torch.equal(vcb.cpu(), vca.cpu())
    e_ref, e_two = oracle.rel_err(out.float().cpu(), ref), oracle.rel_err(out.float().cpu(), two.float().cpu())
    print(f"decode from projection: rel err {e_ref:.3e} (oracle), {e_two:.3e} (two-launch path)")
    assert e_ref <= 2e-2 and e_two <= 1e-2
    # fp32 output: the bf16 output before its rounding
    kcb, vcb = kc0.to(dev), vc0.to(dev)
    o32 = ops.gated_attention_decode_proj(yd, qwd, kwd, kcb, vcb, posd, cosd, sind, num_heads=Hq, splits=splits,
                                          out_dtype=torch.float32)
    assert o32.dtype == torch.float32 and torch.equal(o32.to(torch.bfloat16).cpu(), out.cpu())


# B 2 T 130 (a ragged last key tile), pos0 5 and 3 (cache rows on both sides of the call's), T 1000 (split query
# blocks: the merge kernel reads the gate from y as well), GQA 8 (two head groups per kv head), GQA 1, one token.
@pytest.mark.parametrize("B,T,Hq,Hkv,pos0,max_len", [(2, 130, 8, 2, 0, 192), (1, 70, 8, 2, 5, 128),
                                                     (1, 1000, 8, 2, 0, 1024), (1, 300, 16, 2, 0, 320),
                                                     (1, 96, 4, 4, 3, 128), (1, 1, 8, 2, 0, 64)])
def test_attn_prefill_from_projection(B, T, Hq, Hkv, pos0, max_len):
    """The own-keys prefill from the fused projection output (q35_gated_attn_prefill_proj: q / k norms, RoPE and the
    cache append in the pre-pass, the gate read from y) against the oracle's front end + causal attention, and
    against the two-launch path (q35_attn_prep, then q35_gated_attn_prefill) on the same inputs, whose caches it must
    leave bitwise equal (rows outside pos0 .. pos0 + T - 1 untouched)."""
    dev = device()
    g = torch.Generator().manual_seed(90 + T + Hq)
    D = 256
    y = torch.randn(B, T, Hq * 2 * D + 2 * Hkv * D, generator=g)
    qw, kw = 0.1 * torch.randn(D, generator=g), 0.1 * torch.randn(D, generator=g)
    cos, sin = rope_tables(max_len, rope_inv_freq(D, 0.25, 1e7))
    pos = torch.full((B,), pos0, dtype=torch.int32)
    q, gate, k, v, _ = of.attn_prep(y, qw, kw, cos, sin, pos, Hq, Hkv, D)
    ref = oracle.gated_attention(q, k, v, gate, cos, sin, pos0=pos0)
    kc0 = torch.randn(B, Hkv, max_len, D, generator=g).to(torch.bfloat16)
    vc0 = torch.randn(B, Hkv, max_len, D, generator=g).to(torch.bfloat16)
    announce(f"attn prefill from projection B{B} T{T} Hq{Hq} Hkv{Hkv} pos0 {pos0}")
    yd, qwd, kwd, posd = y.to(dev), qw.to(dev), kw.to(dev), pos.to(dev)
    cosd, sind = cos.to(dev), sin.to(dev)
    kcb, vcb = kc0.to(dev), vc0.to(dev)
    out = ops.gated_attention_prefill_proj(yd, qwd, kwd, kcb, vcb, cosd, sind, num_heads=Hq, pos0=pos0)
    kca, vca = kc0.to(dev), vc0.to(dev)
    qa, ga, ka, va = ops.attn_prep(yd, qwd, kwd, cosd, sind, posd, kca, vca, num_heads=Hq, num_kv_heads=Hkv)
    two = q35hip.gated_attention_prefill(qa, ka, va, ga, cosd, sind, pos0=pos0)
    torch.cuda.synchronize()
    assert torch.equal(kcb.cpu(), kca.cpu()) and torch.equal(vcb.cpu(), vca.cpu())
    e_ref, e_two = oracle.rel_err(out.float().cpu(), ref), oracle.rel_err(out.float().cpu(), two.float().cpu())
    print(f"prefill from projection: rel err {e_ref:.3e} (oracle), {e_two:.3e} (two-launch path)")
    assert out.shape == (B, T, Hq * D) and e_ref <= 2e-2 and e_two <= 1e-2


# Rows at different positions (0, mid-cache, the last rows), ragged key ranges, GQA 1 / 4 / 8, one token.
@pytest.mark.parametrize("B,T,Hq,Hkv,max_len,pos", [(3, 100, 8, 2, 448, [0, 37, 300]), (2, 1, 8, 2, 256, [5, 255]),
                                                     (1, 257, 4, 4, 640, [383]), (2, 64, 8, 1, 192, [128, 0]),
                                                     (1, 130, 16, 2, 320, [64])])
def test_attn_prefill_over_cache_from_projection(B, T, Hq, Hkv, max_len, pos):
    """The multi-token call over the cache from the fused projection output (q35_gated_attn_prefill_cached_proj: the
    front end and the cache append in the pre-pass, whose value blocks take the earlier rows from the cache and the
    call's rows from y) against the oracle's front end + cached attention, and against q35_attn_prep +
    q35_gated_attn_prefill_cached on the same inputs, whose caches it must leave bitwise equal."""
    dev = device()
    g = torch.Generator().manual_seed(70 + T + max_len)
    D = 256
    y = torch.randn(B, T, Hq * 2 * D + 2 * Hkv * D, generator=g)
    qw, kw = 0.1 * torch.randn(D, generator=g), 0.1 * torch.randn(D, generator=g)
    cos, sin = rope_tables(max_len, rope_inv_freq(D, 0.25, 1e7))
    pos_t = torch.tensor(pos, dtype=torch.int32)
    kc0 = torch.randn(B, Hkv, max_len, D, generator=g).to(torch.bfloat16)
    vc0 = torch.randn(B, Hkv, max_len, D, generator=g).to(torch.bfloat16)
    q, gate, _, v, k_rot = of.attn_prep(y, qw, kw, cos, sin, pos_t, Hq, Hkv, D)
    kr, vr = kc0.clone(), vc0.clone()
    for b in range(B):
        p0 = int(pos_t[b])
        kr[b, :, p0:p0 + T] = k_rot[b].transpose(0, 1).to(torch.bfloat16)
        vr[b, :, p0:p0 + T] = v[b].transpose(0, 1).to(torch.bfloat16)
    ref = oracle.gated_attention_cached(q, kr, vr, gate, pos_t, cos, sin)
    announce(f"attn prefill over cache from projection B{B} T{T} Hq{Hq} Hkv{Hkv} max_len {max_len} pos {pos}")
    yd, qwd, kwd, posd = y.to(dev), qw.to(dev), kw.to(dev), pos_t.to(dev)
    cosd, sind = cos.to(dev), sin.to(dev)
    kcb, vcb = kc0.to(dev), vc0.to(dev)
    out = ops.gated_attention_prefill_cached_proj(yd, qwd, kwd, kcb, vcb, posd, cosd, sind, num_heads=Hq)
    kca, vca = kc0.to(dev), vc0.to(dev)
    qa, ga, _, _ = ops.attn_prep(yd, qwd, kwd, cosd, sind, posd, kca, vca, num_heads=Hq, num_kv_heads=Hkv,
                                 want_kv=False)
    two = ops.gated_attention_prefill_cached(qa, kca, vca, ga, posd, cosd, sind)
    torch.cuda.synchronize()
    assert torch.equal(kcb.cpu(), kca.cpu()) and torch.equal(vcb.cpu(), vca.cpu())
    # values: the fp32 rows rounded to bf16, bitwise the oracle's; keys: one bf16 rounding of the fp32 front end
    assert torch.equal(vcb.cpu(), vr) and oracle.rel_err(kcb.cpu().float(), kr.float()) <= TOL_BF16
    e_ref, e_two = oracle.rel_err(out.float().cpu(), ref), oracle.rel_err(out.float().cpu(), two.float().cpu())
    print(f"prefill over cache from projection: rel err {e_ref:.3e} (oracle), {e_two:.3e} (two-launch path)")
    assert out.shape == (B, T, Hq * D) and e_ref <= 2e-2 and e_two <= 1e-2


@pytest.mark.parametrize("with_add", [False, True])
def test_add_rmsnorm_matches_oracle(with_add):
    """Residual add + RMSNorm(1 + w) (HF:720-734): x updated in place, h returned."""
    from oracle import model as om
    dev = device()
    g = torch.Generator().manual_seed(70)
    x = torch.randn(3, 5, 1024, generator=g)
    y = torch.randn(3, 5, 1024, generator=g) if with_add else None
    w = 0.1 * torch.randn(1024, generator=g)
    xs = x + y if with_add else x
    ref = om.rmsnorm_1p(xs, w, 1e-6)
    announce(f"add_rmsnorm add={with_add}")
    xd = x.to(dev)
    h = ops.add_rmsnorm_(xd, None if y is None else y.to(dev), w.to(dev))
    torch.cuda.synchronize()
    assert oracle.rel_err(h.cpu(), ref) <= TOL_F32
    assert oracle.rel_err(xd.cpu(), xs) <= TOL_F32


@pytest.mark.parametrize("with_scale", [False, True])
def test_gated_rmsnorm_split_output(with_scale):
    """The gated norm with its output in the int8 GEMM's split layout (the GDN output projection's input): equal to
    ops.split_activations of the fp32 form's output, bitwise, z rows strided as in the fused projection output."""
    dev = device()
    g = torch.Generator().manual_seed(72)
    M, Hv = 70, 16
    o = torch.randn(M, Hv, 128, generator=g).to(dev)
    zw = torch.randn(M, Hv * 128 + 40, generator=g).to(dev)
    w = (1.0 + 0.1 * torch.randn(128, generator=g)).to(dev)
    hs = (1.0 + 0.1 * torch.randn(Hv, generator=g)).to(dev) if with_scale else None
    announce(f"gated_rmsnorm split scale={with_scale}")
    a = ops.gated_rmsnorm(o, zw[:, 8:8 + Hv * 128], w, hs)
    b = ops.gated_rmsnorm(o, zw[:, 8:8 + Hv * 128], w, hs, split=True)
    torch.cuda.synchronize()
    assert b.dtype == torch.int32 and b.shape == a.shape
    assert torch.equal(b, ops.split_activations(a))


def test_gated_rmsnorm_aligned_and_unaligned_forms():
    """16-byte-aligned o and z take the two-heads-per-wave form, a z one float off alignment the one-head form: the
    two agree to fp32 rounding (only the summation order of the squares differs), fp32 and bf16, and each one's split
    output equals ops.split_activations of its fp32 output."""
    dev = device()
    g = torch.Generator().manual_seed(73)
    M, Hv = 37, 16
    o = torch.randn(M, Hv, 128, generator=g).to(dev)
    zw = torch.randn(M, Hv * 128 + 12, generator=g).to(dev)
    w = (1.0 + 0.1 * torch.randn(128, generator=g)).to(dev)
    announce("gated_rmsnorm aligned / unaligned z")
    za, zu = zw[:, 8:8 + Hv * 128], zw[:, 9:9 + Hv * 128]
    for dt in (torch.float32, torch.bfloat16):
        a = ops.gated_rmsnorm(o.to(dt), zu, w).float()
        b = ops.gated_rmsnorm(o.to(dt), zu.contiguous(), w).float()
        torch.cuda.synchronize()
        assert oracle.rel_err(a.cpu(), b.cpu()) <= (1e-6 if dt == torch.float32 else 1e-2)
    for z in (za, zu):
        f = ops.gated_rmsnorm(o, z, w)
        assert torch.equal(ops.gated_rmsnorm(o, z, w, split=True), ops.split_activations(f))


@pytest.mark.parametrize("with_add,H", [(False, 1024), (True, 1024), (True, 1000)])
def test_add_rmsnorm_split_output(with_add, H):
    """The norm with its output in the int8 GEMM's split layout: the words equal ops.split_activations of the fp32
    output (the same norm, then hi = bf16(h), lo = bf16(h - hi)), and x is updated as by the fp32 form."""
    dev = device()
    g = torch.Generator().manual_seed(71)
    x = torch.randn(3, 7, H, generator=g).to(dev)
    y = torch.randn(3, 7, H, generator=g).to(dev) if with_add else None
    w = (0.1 * torch.randn(H, generator=g)).to(dev)
    announce(f"add_rmsnorm split add={with_add} H{H}")
    xa, xb = x.clone(), x.clone()
    h = ops.add_rmsnorm_(xa, y, w)
    hs = ops.add_rmsnorm_(xb, y, w, split=True)
    torch.cuda.synchronize()
    assert hs.dtype == torch.int32 and hs.shape == h.shape
    assert torch.equal(hs, ops.split_activations(h))
    assert torch.equal(xa, xb)


@pytest.mark.parametrize("with_bias,with_scale", [(False, False), (True, True)])
def test_gdn_decode_fused_equals_the_three_kernels(with_bias, with_scale):
    """Five decode steps through q35_gdn_decode_fused (conv + recurrent rule + gated norm in one launch) against the
    same steps through gdn_conv, gdn_decode_step_ and gated_rmsnorm: the conv state is bitwise equal at every step,
    the outputs and the recurrent state agree to fp32 rounding (relative error <= 1e-6: the same arithmetic with the
    same reduction order; the compiler may contract a multiply-add differently in the two builds), and the fused
    output matches the CPU oracle's conv + recurrence + gated norm within the fp32 tolerance."""
    dev = device()
    B, H, d, K = 3, 16, 128, 4
    y, conv_w, cstate, A_log, dt_bias, C, W = _gdn_case(B, 5, seed=61)
    gen = torch.Generator().manual_seed(62)
    bias = torch.randn(C, generator=gen) if with_bias else None
    hs = (0.5 + torch.rand(H, generator=gen)) if with_scale else None
    nw = 1.0 + 0.1 * torch.randn(d, generator=gen)
    S0 = 0.1 * torch.randn(B, H, d, d, generator=gen)
    Vd = H * d
    b_off, a_off, z_off = C + Vd, C + Vd + H, C
    todev = (lambda t: None if t is None else t.to(dev))
    cs_f, cs_u = cstate.to(dev), cstate.to(dev)
    S_f, S_u = S0.to(dev), S0.to(dev)
    cw, Al, dt, nwd, hsd, bd = conv_w.to(dev), A_log.to(dev), dt_bias.to(dev), nw.to(dev), todev(hs), todev(bias)
    # CPU oracle of the same steps
    cs_r, S_r = cstate.clone(), S0.clone()
    for t in range(5):
        announce(f"gdn_decode_fused step {t} bias {with_bias} head_scale {with_scale}")
        yt = y[:, t:t + 1].contiguous()
        ytd = yt.to(dev)
        out_f = ops.gdn_decode_fused_(ytd.view(B, W), cw, cs_f, Al, dt, S_f, nwd, b_off=b_off, a_off=a_off,
                                      z_off=z_off, head_scale=hsd, conv_bias=bd)
        q, k, v, g, beta = ops.gdn_conv(ytd, cw, cs_u, Al, dt, num_k_heads=H, head_k_dim=d, num_v_heads=H,
                                        head_v_dim=d, b_off=b_off, a_off=a_off, conv_bias=bd)
        o = ops.gdn_decode_step_(q, k, v, g, beta, S_u, use_qk_l2norm_in_kernel=True)
        out_u = ops.gated_rmsnorm(o, ytd[..., z_off:z_off + Vd], nwd, hsd, 1e-6)
        torch.cuda.synchronize()
        assert oracle.rel_err(out_f.cpu(), out_u.view(B, Vd).cpu()) <= 1e-6, f"step {t}: output"
        assert torch.equal(cs_f.cpu(), cs_u.cpu()), f"step {t}: conv state differs"
        assert oracle.rel_err(S_f.cpu(), S_u.cpu()) <= 1e-6, f"step {t}: recurrent state"
        qr, kr, vr, gr, br, cs_r = of.gdn_conv(yt, conv_w, cs_r, A_log, dt_bias, H, d, H, d, b_off, a_off,
                                               conv_bias=bias)
        o_r, S_r = oracle.recurrent_gated_delta_rule(qr, kr, vr, gr, br, initial_state=S_r,
                                                     output_final_state=True, use_qk_l2norm_in_kernel=True)
        ref = of.gated_rmsnorm(o_r, yt[..., z_off:z_off + Vd], nw, hs, 1e-6)
        assert oracle.rel_err(out_f.cpu(), ref.reshape(B, Vd)) <= TOL_F32
    assert oracle.rel_err(S_f.cpu(), S_r) <= TOL_F32
