"""The GDN decode step split over three kernels (the decode GEMVs' conv epilogue and gated-norm prologue around the
four-blocks-per-head recurrent kernel) against the one-launch fused step and the CPU oracle.

Tolerances (relative error): the same fp32 arithmetic in the same reduction order as the fused step <= 1e-6 (the
compiler may contract a multiply-add differently); the gated norm formed per head in the GEMV's staging (a different
summation order of the squares) and the split-K products' atomic additions <= 1e-5, the fp32 bound of these tests.
"""
import pytest
import torch

import oracle
from oracle import frontend as of
from oracle import mlp as omlp
from q35hip import layers, ops
from q35hip.workloads import quantize_int8, dequantize_int8
from gpu_util import announce, device

pytestmark = pytest.mark.gpu

TOL_SAME = 1e-6
TOL_F32 = 1e-5


def _case(B, H, seed, K=4, d=128):
    g = torch.Generator().manual_seed(seed)
    C = 3 * H * d
    W = C + H * d + 2 * H  # [qkv | z | b | a]
    y = torch.randn(B, 5, W, generator=g)
    conv_w = 0.5 * torch.randn(C, K, generator=g)
    cstate = torch.randn(B, K - 1, C, generator=g)
    A_log = torch.log(torch.rand(H, generator=g) * 16)
    dt_bias = torch.ones(H) + 0.1 * torch.randn(H, generator=g)
    S0 = 0.1 * torch.randn(B, H, d, d, generator=g)
    nw = 1.0 + 0.1 * torch.randn(d, generator=g)
    hs = 0.5 + torch.rand(H, generator=g)
    return y, conv_w, cstate, A_log, dt_bias, S0, nw, hs, C, W


def test_sliced_recurrent_step_equals_the_fused_step():
    """Five steps: the fused step against gdn_conv (T = 1, written back into the projection row as the conv epilogue
    does) + the sliced recurrent kernel + gated_rmsnorm. Outputs and states agree to fp32 rounding (same arithmetic,
    same column-sum order); the sliced kernel's output also matches the CPU oracle's recurrence."""
    dev = device()
    B, H, d = 3, 16, 128
    y, conv_w, cstate, A_log, dt_bias, S0, nw, hs, C, W = _case(B, H, seed=71)
    Vd = H * d
    b_off, a_off, z_off = C + Vd, C + Vd + H, C
    cw, Al, dt, nwd, hsd = conv_w.to(dev), A_log.to(dev), dt_bias.to(dev), nw.to(dev), hs.to(dev)
    cs_f, cs_s = cstate.to(dev), cstate.to(dev)
    S_f, S_s = S0.to(dev), S0.to(dev)
    S_r, cs_r = S0.clone(), cstate.clone()
    for t in range(5):
        announce(f"gdn decode sliced step {t}")
        yt = y[:, t].contiguous()
        ytd = yt.to(dev)
        out_f = ops.gdn_decode_fused_(ytd, cw, cs_f, Al, dt, S_f, nwd, b_off=b_off, a_off=a_off, z_off=z_off,
                                      head_scale=hsd)
        q, k, v, g, beta = ops.gdn_conv(ytd.view(B, 1, W), cw, cs_s, Al, dt, num_k_heads=H, head_k_dim=d,
                                        num_v_heads=H, head_v_dim=d, b_off=b_off, a_off=a_off)
        yc = ytd.clone()
        yc[:, :C] = torch.cat([q.reshape(B, -1), k.reshape(B, -1), v.reshape(B, -1)], dim=1)
        o = ops.gdn_decode_sliced_(yc, Al, dt, S_s, b_off=b_off, a_off=a_off)
        out_s = ops.gated_rmsnorm(o.view(B, 1, H, d), yc.view(B, 1, W)[..., z_off:z_off + Vd], nwd, hsd, 1e-6)
        torch.cuda.synchronize()
        assert oracle.rel_err(out_s.view(B, Vd).cpu(), out_f.cpu()) <= TOL_SAME, f"step {t}: output"
        assert oracle.rel_err(S_s.cpu(), S_f.cpu()) <= TOL_SAME, f"step {t}: state"
        qr, kr, vr, gr, br, cs_r = of.gdn_conv(yt[:, None], conv_w, cs_r, A_log, dt_bias, H, d, H, d, b_off, a_off)
        o_r, S_r = oracle.recurrent_gated_delta_rule(qr, kr, vr, gr, br, initial_state=S_r, output_final_state=True,
                                                     use_qk_l2norm_in_kernel=True)
        assert oracle.rel_err(o.cpu(), o_r.reshape(B, Vd)) <= TOL_F32, f"step {t}: raw output vs oracle"
    assert oracle.rel_err(S_s.cpu(), S_r) <= TOL_F32


@pytest.mark.parametrize("group", [128, 0])
@pytest.mark.parametrize("with_bias", [False, True])
def test_gemv_conv_epilogue_equals_gemv_then_conv(group, with_bias):
    """The input projection with the residual add + norm prologue and the conv epilogue against the same GEMV
    followed by gdn_conv at T = 1: the convolved channels, the other channels and the advanced conv state agree to
    fp32 rounding (the two kernel variants may contract a multiply-add differently), the residual sum bit for bit
    (N 2056: a ragged last tile)."""
    dev = device()
    B, H, d, Kh = 3, 4, 128, 1024
    C = 3 * H * d
    N = C + H * d + 2 * H
    g = torch.Generator().manual_seed(81 + group + with_bias)
    q, s = quantize_int8(torch.randn(N, Kh, generator=g) * 0.05, group)
    x = torch.randn(B, Kh, generator=g)
    xa = torch.randn(B, Kh, generator=g)
    nwn = 0.1 * torch.randn(Kh, generator=g)
    conv_w = 0.5 * torch.randn(C, 4, generator=g)
    bias = torch.randn(C, generator=g) if with_bias else None
    cstate = torch.randn(B, 3, C, generator=g)
    A_log = torch.zeros(H)
    dt_bias = torch.ones(H)
    announce(f"gemv conv epilogue group {group} bias {with_bias}")
    qd, sd, xd, xad, nwd, cwd = q.to(dev), s.to(dev), x.to(dev), xa.to(dev), nwn.to(dev), conv_w.to(dev)
    bd = None if bias is None else bias.to(dev)
    cs_a, cs_b = cstate.to(dev), cstate.to(dev)
    xo_a, xo_b = torch.empty(B, Kh, device=dev), torch.empty(B, Kh, device=dev)
    y_a = ops.gemv(xd, qd, sd, prenorm=(xad, nwd, 1e-6, xo_a), conv=(cwd, bd, cs_a))
    y_b = ops.gemv(xd, qd, sd, prenorm=(xad, nwd, 1e-6, xo_b))
    qc, kc, vc, _, _ = ops.gdn_conv(y_b.view(B, 1, N), cwd, cs_b, A_log.to(dev), dt_bias.to(dev), num_k_heads=H,
                                    head_k_dim=d, num_v_heads=H, head_v_dim=d, b_off=C + H * d,
                                    a_off=C + H * d + H, conv_bias=bd)
    torch.cuda.synchronize()
    conv_ref = torch.cat([qc.reshape(B, -1), kc.reshape(B, -1), vc.reshape(B, -1)], dim=1)
    assert oracle.rel_err(y_a[:, :C].cpu(), conv_ref.cpu()) <= TOL_SAME
    assert oracle.rel_err(y_a[:, C:].cpu(), y_b[:, C:].cpu()) <= TOL_SAME
    assert oracle.rel_err(cs_a.cpu(), cs_b.cpu()) <= TOL_SAME
    assert torch.equal(xo_a.cpu(), xo_b.cpu())
    # and against the CPU oracle: RMSNorm (1 + w) of x + x_add, the q8 product, the conv
    hs = x + xa
    hn = hs * torch.rsqrt(hs.pow(2).mean(-1, keepdim=True) + 1e-6) * (1.0 + nwn)
    yr = omlp.q8_linear(hn, q, s)
    qr, kr, vr, _, _, cs_r = of.gdn_conv(yr[:, None], conv_w, cstate, A_log, dt_bias, H, d, H, d, C + H * d,
                                         C + H * d + H, conv_bias=bias)
    ref = torch.cat([qr.reshape(B, -1), kr.reshape(B, -1), vr.reshape(B, -1)], dim=1)
    assert oracle.rel_err(y_a[:, :C].cpu(), ref) <= TOL_F32
    assert oracle.rel_err(cs_a.cpu(), cs_r) <= TOL_F32


@pytest.mark.parametrize("group", [128, 0])
@pytest.mark.parametrize("epilogue", ["store", "add"])
@pytest.mark.parametrize("with_scale", [False, True])
def test_gemv_gated_norm_prologue(group, epilogue, with_scale):
    """The output projection with the gated RMSNorm in its staging against gated_rmsnorm + gemv and against the CPU
    oracle (K 2048 = 16 heads; the add epilogue splits K over four blocks per 16 rows; z a strided view of a wider
    projection row)."""
    dev = device()
    M, H, d, N = 3, 16, 128, 1024
    K = H * d
    g = torch.Generator().manual_seed(91 + group + 2 * with_scale + (epilogue == "add"))
    q, s = quantize_int8(torch.randn(N, K, generator=g) * 0.05, group)
    o = torch.randn(M, K, generator=g)
    zrow = torch.randn(M, K + 40, generator=g)  # z is columns 8 .. 8 + K of a wider row
    nw = 1.0 + 0.1 * torch.randn(d, generator=g)
    hs = (0.5 + torch.rand(H, generator=g)) if with_scale else None
    base = torch.randn(M, N, generator=g)
    announce(f"gemv gated norm group {group} {epilogue} scale {with_scale}")
    od, zd = o.to(dev), zrow.to(dev)[:, 8:]
    qd, sd, nwd = q.to(dev), s.to(dev), nw.to(dev)
    hsd = None if hs is None else hs.to(dev)
    out = base.to(dev) if epilogue == "add" else torch.empty(M, N, device=dev)
    ops.gemv_gated_norm(od, zd, nwd, qd, sd, out, head_scale=hsd, epilogue=epilogue)
    xn = ops.gated_rmsnorm(od.view(M, 1, H, d), zd.reshape(M, 1, -1)[..., :K].contiguous(), nwd, hsd, 1e-6)
    ref_d = ops.gemv(xn.view(M, K).contiguous(), qd, sd)
    torch.cuda.synchronize()
    expect = ref_d.cpu() + (base if epilogue == "add" else 0)
    assert oracle.rel_err(out.cpu(), expect) <= TOL_F32
    xr = of.gated_rmsnorm(o.view(M, 1, H, d), zrow[:, 8:8 + K].reshape(M, 1, K), nw, hs, 1e-6).reshape(M, K)
    ref = omlp.q8_linear(xr, q, s) + (base if epilogue == "add" else 0)
    assert oracle.rel_err(out.cpu(), ref) <= TOL_F32


def test_gdn_layer_decode_on_int8_projections_equals_the_fused_composition():
    """gated_deltanet_layer at T = 1 with int8 projections (the split path: conv epilogue, sliced recurrence, gated
    norm prologue) against the same step composed from the fused kernel and plain GEMVs, over three steps with the
    residual add: residual and both states agree within the fp32 bound."""
    dev = device()
    B, Hd, Hv, d, K = 3, 1024, 16, 128, 4
    C, Vd = 3 * Hv * d, Hv * d
    g = torch.Generator().manual_seed(101)
    p = {}
    for name, (o_, i_) in (("in_proj_qkv", (C, Hd)), ("in_proj_z", (Vd, Hd)), ("in_proj_b", (Hv, Hd)),
                           ("in_proj_a", (Hv, Hd)), ("out_proj", (Hd, Vd))):
        qq, ss = quantize_int8(torch.randn(o_, i_, generator=g) * 0.05, 128)
        p[name + ".q"], p[name + ".s"], p[name] = qq, ss, dequantize_int8(qq, ss)
    p["conv1d"] = 0.5 * torch.randn(C, K, generator=g)
    p["A_log"] = torch.log(torch.rand(Hv, generator=g) * 16)
    p["dt_bias"] = torch.ones(Hv)
    p["norm"] = 1.0 + 0.1 * torch.randn(d, generator=g)
    pd = {k: v.to(dev) for k, v in p.items()}
    ln_w = (0.1 * torch.randn(Hd, generator=g)).to(dev)
    hs = (0.5 + torch.rand(Hv, generator=g)).to(dev)
    cs0 = torch.randn(B, K - 1, C, generator=g)
    S0 = 0.1 * torch.randn(B, Hv, d, d, generator=g)
    res0 = torch.randn(B, 1, Hd, generator=g)
    cs_a, cs_b = cs0.to(dev), cs0.to(dev)
    S_a, S_b = S0.to(dev), S0.to(dev)
    res_a, res_b = res0.to(dev), res0.to(dev)
    for t in range(3):
        announce(f"gdn layer decode split vs fused step {t}")
        layers.gated_deltanet_layer(res_a, pd, cs_a, S_a, head_scale=hs, prenorm=(None, ln_w, 1e-6, None),
                                    residual=res_a)
        # the fused composition: input GEMV with the norm prologue, fused step, output GEMV adding into the residual
        w_in = layers.gdn_in_weight(pd)
        y = layers.linear(res_b, w_in, *layers._q8(pd, "_in_fused"), prenorm=(None, ln_w, 1e-6, None))
        o = ops.gdn_decode_fused_(y.view(B, -1), pd["conv1d"], cs_b, pd["A_log"], pd["dt_bias"], S_b, pd["norm"],
                                  b_off=C + Vd, a_off=C + Vd + Hv, z_off=C, head_scale=hs)
        layers.linear(o.view(B, 1, Vd), pd["out_proj"], *layers._q8(pd, "out_proj"), residual=res_b)
        torch.cuda.synchronize()
        assert oracle.rel_err(res_a.cpu(), res_b.cpu()) <= TOL_F32, f"step {t}: residual"
        assert oracle.rel_err(S_a.cpu(), S_b.cpu()) <= TOL_F32, f"step {t}: state"
        assert oracle.rel_err(cs_a.cpu(), cs_b.cpu()) <= TOL_SAME, f"step {t}: conv state"
