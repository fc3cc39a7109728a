"""Decode matrix-vector products (int8 per-output-channel and fp32 weights) and the SwiGLU neuron hook on the GPU,
against the CPU oracle. fp32 arithmetic throughout: relative error <= 1e-5 (summation order only)."""
import pytest
import torch

import oracle
from oracle import mlp as omlp
import q35hip
from q35hip import ops
from gpu_util import announce, device

pytestmark = pytest.mark.gpu

TOL = 1e-5


def _weights(N, K, wdt, seed):
    g = torch.Generator().manual_seed(seed)
    if wdt == torch.int8:
        return torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8), torch.rand(N, generator=g) * 0.01
    return torch.randn(N, K, generator=g) * 0.05, None


@pytest.mark.parametrize("wdt", [torch.int8, torch.float32])
@pytest.mark.parametrize("M,N,K", [(1, 1024, 1024), (3, 7168, 1024), (3, 1024, 3584), (8, 1000, 2048),
                                   (5, 2048, 256), (3, 20000, 1024)])
def test_gemv_store_and_add(wdt, M, N, K):
    """Per-row int8 and fp32 weights, store and accumulate. N 20000 has more 16-row tiles than blocks, so blocks
    loop over tiles (one K step per wave with int8 at K 1024, four with fp32)."""
    dev = device()
    W, s = _weights(N, K, wdt, seed=N + K)
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(M))
    ref = omlp.q8_linear(x, W, s) if wdt == torch.int8 else x @ W.T
    announce(f"gemv {wdt} M{M} N{N} K{K}")
    Wd, sd, xd = W.to(dev), None if s is None else s.to(dev), x.to(dev)
    y = ops.gemv(xd, Wd, sd)
    base = torch.randn(M, N, generator=torch.Generator().manual_seed(9))
    acc = base.to(dev)
    ops.gemv(xd, Wd, sd, out=acc, epilogue="add")
    torch.cuda.synchronize()
    assert oracle.rel_err(y.cpu(), ref) <= TOL
    assert oracle.rel_err(acc.cpu(), base + ref) <= TOL


@pytest.mark.parametrize("M,T", [(3, 1), (6, 2)])
def test_gemv_swiglu_with_pushes_and_prefill_form(M, T):
    """Interleaved (gate, up) int8 rows through the SwiGLU epilogue, with add / mul / all-neuron pushes; the prefill
    form (swiglu_push over a [gate | up] projection) gives the same activations."""
    dev = device()
    I, H = 3584, 1024
    Wg, sg = _weights(I, H, torch.int8, 1)
    Wu, su = _weights(I, H, torch.int8, 2)
    x = torch.randn(M, H, generator=torch.Generator().manual_seed(3))
    pushes = [(17, "add", [1.5, -2.0, 0.25]), (17, "mul", [3.0, 0.5]), (None, "mul", [1.0, 0.75, 1.25]),
              (3583, "add", [4.0])]
    ref = omlp.swiglu_push(omlp.q8_linear(x, Wg, sg), omlp.q8_linear(x, Wu, su), pushes, T=T)
    Wi = torch.stack([Wg, Wu], dim=1).reshape(2 * I, H)          # row 2 j gate j, row 2 j + 1 up j
    si = torch.stack([sg, su], dim=1).reshape(2 * I)
    announce(f"gemv swiglu M{M} T{T}")
    pk = ops.pack_pushes(pushes, dev)
    a = ops.gemv(x.to(dev), Wi.to(dev), si.to(dev), epilogue="swiglu", pushes=pk, T=T)
    gu = torch.cat([omlp.q8_linear(x, Wg, sg), omlp.q8_linear(x, Wu, su)], dim=-1)
    a2 = ops.swiglu_push(gu.to(dev), pk, T=T)
    torch.cuda.synchronize()
    assert oracle.rel_err(a.cpu(), ref) <= TOL
    assert oracle.rel_err(a2.cpu(), ref) <= TOL


@pytest.mark.parametrize("rows,n", [(1, 151936), (3, 151936), (2, 1000), (5, 4099)])
def test_argmax_rows_matches_torch(rows, n):
    """Device argmax (engine/kernels.js:260-283) against torch.argmax, with planted ties (the lowest index wins) and
    rows of -inf."""
    dev = device()
    g = torch.Generator().manual_seed(n + rows)
    x = torch.randn(rows, n, generator=g)
    x[0, 7] = x[0, n - 2] = x[0].max() + 1.0          # a tie: index 7 must win
    if rows > 1:
        x[1] = -float("inf")                          # all -inf: index 0
    if rows > 2:
        x[2, n - 1] = 1e30                            # the last element (a tail element when n % 4 != 0)
    announce(f"argmax rows{rows} n{n}")
    got = ops.argmax_rows(x.to(dev))
    torch.cuda.synchronize()
    assert got.dtype == torch.int32
    assert torch.equal(got.cpu().long(), x.argmax(-1))
    # rows that start 4 bytes past a 16-byte boundary and have a row stride of n + 1 (every row a different head
    # of scalar elements before the 16-byte loads)
    # (through the C ABI, which takes the row stride)
    base = torch.full((rows, n + 1), -5.0)
    base[:, 1:] = x
    based = base.to(dev)
    got2 = torch.full((rows,), -1, dtype=torch.int32, device=dev)
    st = q35hip.lib().q35_argmax_rows(based.data_ptr() + 4, n + 1, rows, n, got2.data_ptr(), None,
                                      torch.cuda.current_stream().cuda_stream)
    assert st == 0
    torch.cuda.synchronize()
    assert torch.equal(got2.cpu().long(), x.argmax(-1))


@pytest.mark.parametrize("M,N,K,fmt", [(3, 151936, 1024, "g128"), (1, 40008, 1024, "g128"), (2, 5000, 1024, "row"),
                                       (8, 20000, 2048, "g128"), (2, 20000, 1024, "f32")])
def test_gemv_norm_argmax_matches_torch(M, N, K, fmt):
    """The LM head's GEMV with the greedy pick folded in (q35_gemv_norm_argmax): the logits bitwise those of the plain
    norm GEMV, each row's index torch.argmax of them (two identical weight rows planted as the largest logit of row 0:
    the lower index wins), and the slots left zero for the next call (second call on other inputs). The shapes run the
    block tile loop (N 151936, 40008, 20000; int8 and fp32 weights) and one tile per block (N 5000)."""
    dev = device()
    g = torch.Generator().manual_seed(N + M)
    Wf = torch.randn(N, K, generator=g) * 0.02
    x = torch.randn(M, K, generator=g)
    nw = torch.randn(K, generator=g) * 0.1
    h = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6) * (1.0 + nw)
    lo, hi = N // 7, N - 3
    Wf[lo] = h[0] / h[0].norm() * 0.5   # the largest logit of row 0, twice
    Wf[hi] = Wf[lo]
    if fmt == "g128":
        W, s = omlp.q8_quantize(Wf)
    elif fmt == "f32":
        W, s = Wf, None
    else:
        amax = Wf.abs().amax(1).clamp_min(1e-12)
        s = amax / 127
        W = torch.round(Wf / s[:, None]).clamp(-127, 127).to(torch.int8)
    announce(f"gemv norm argmax M{M} N{N} K{K} {fmt}")
    Wd, sd, nwd = W.to(dev), None if s is None else s.to(dev), nw.to(dev)
    slots = torch.zeros(M, dtype=torch.int64, device=dev)
    for call in range(2):
        xc = x if call == 0 else torch.randn(M, K, generator=g)
        xd = xc.to(dev)
        y, idx = ops.gemv_norm_argmax(xd, Wd, sd, (None, nwd, 1e-6, None), slots)
        plain = ops.gemv(xd, Wd, sd, prenorm=(None, nwd, 1e-6, None))
        torch.cuda.synchronize()
        assert torch.equal(y.cpu(), plain.cpu())
        assert torch.equal(idx.cpu().long(), y.cpu().argmax(-1))
        assert int(slots.abs().sum()) == 0
        if call == 0:
            assert int(idx[0]) == lo


@pytest.mark.parametrize("epilogue", ["store", "add", "swiglu"])
@pytest.mark.parametrize("with_add,with_out", [(False, False), (True, True), (True, False)])
def test_gemv_with_fused_residual_add_and_rmsnorm(epilogue, with_add, with_out):
    """q35_gemv_norm: the product of RMSNorm(1 + w) of x + x_add (HF:720-734 after the residual add) equals the oracle's
    norm followed by the plain product; x + x_add lands in x_out."""
    from oracle import model as om
    dev = device()
    M, H = 3, 1024
    N = 2048 if epilogue == "swiglu" else 1536
    W, s = _weights(N, H, torch.int8, 77)
    g = torch.Generator().manual_seed(78)
    x = torch.randn(M, H, generator=g)
    xa = torch.randn(M, H, generator=g) if with_add else None
    nw = 0.3 * torch.randn(H, generator=g)
    ssum = x + xa if with_add else x
    h = om.rmsnorm_1p(ssum, nw, 1e-6)
    lin = omlp.q8_linear(h, W, s)
    if epilogue == "swiglu":
        ref = torch.nn.functional.silu(lin[:, 0::2]) * lin[:, 1::2]
    else:
        ref = lin
    base = torch.randn(ref.shape, generator=g)
    announce(f"gemv_norm {epilogue} add={with_add} out={with_out}")
    xd = x.to(dev)
    xo = torch.full((M, H), 5.0, device=dev) if with_out else None
    out = base.to(dev) if epilogue == "add" else None
    y = ops.gemv(xd, W.to(dev), s.to(dev), out=out, epilogue=epilogue,
                 prenorm=(None if xa is None else xa.to(dev), nw.to(dev), 1e-6, xo))
    torch.cuda.synchronize()
    exp = base + ref if epilogue == "add" else ref
    assert oracle.rel_err(y.cpu(), exp) <= TOL
    assert torch.equal(xd.cpu(), x)  # the residual itself is only read
    if with_out:
        assert oracle.rel_err(xo.cpu(), ssum) <= 1e-7


def _weights_g128(N, K, seed):
    """int8 weights with one scale per group of 128 inputs (the engine's q8 format), the scales of neighbouring groups
    a decade apart so that a scale applied to the wrong group shows."""
    g = torch.Generator().manual_seed(seed)
    q = torch.randint(-127, 128, (N, K), generator=g, dtype=torch.int8)
    s = torch.rand(N, K // 128, generator=g) * 0.01 * (10.0 ** (torch.arange(K // 128) % 2))[None, :]
    return q, s


@pytest.mark.parametrize("M,N,K", [(1, 8224, 1024), (3, 1024, 3584), (3, 1024, 2048), (8, 1000, 2048),
                                   (2, 4096, 4352), (3, 5000, 1024), (3, 40008, 1024), (2, 17000, 3584)])
def test_gemv_group_scales_store_add_and_norm(M, N, K):
    """Q35_I8_G128 weights: store, accumulate, and the fused residual add + RMSNorm prologue, against the oracle's
    per-group dequantised product (K 4352 takes the four-steps-per-wave form; N 5000 a ragged last tile; N 40008 and
    17000 more 16-row tiles than blocks, so blocks loop over tiles, with one and two K steps per wave)."""
    dev = device()
    W, s = _weights_g128(N, K, seed=N + K)
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(M))
    ref = omlp.q8_linear(x, W, s)
    announce(f"gemv g128 M{M} N{N} K{K}")
    Wd, sd, xd = W.to(dev), s.to(dev), x.to(dev)
    y = ops.gemv(xd, Wd, sd)
    base = torch.randn(M, N, generator=torch.Generator().manual_seed(9))
    acc = base.to(dev)
    ops.gemv(xd, Wd, sd, out=acc, epilogue="add")
    xa = torch.randn(M, K, generator=torch.Generator().manual_seed(10))
    nw = torch.randn(K, generator=torch.Generator().manual_seed(11)) * 0.1
    xs = torch.empty(M, K, device=dev)
    yn = ops.gemv(xd, Wd, sd, prenorm=(xa.to(dev), nw.to(dev), 1e-6, xs))
    hs = x + xa
    hn = hs * torch.rsqrt(hs.pow(2).mean(-1, keepdim=True) + 1e-6) * (1.0 + nw)
    torch.cuda.synchronize()
    assert oracle.rel_err(y.cpu(), ref) <= TOL
    assert oracle.rel_err(acc.cpu(), base + ref) <= TOL
    assert oracle.rel_err(yn.cpu(), omlp.q8_linear(hn, W, s)) <= TOL
    assert torch.equal(xs.cpu(), hs)


@pytest.mark.parametrize("I", [3584, 12000])
def test_gemv_group_scales_swiglu_with_pushes(I):
    """Interleaved (gate, up) rows with interleaved group scales through the SwiGLU + push epilogue (I 12000: 1500
    16-row tiles looped over the blocks)."""
    dev = device()
    H, M = 1024, 3
    Wg, sg = _weights_g128(I, H, 21)
    Wu, su = _weights_g128(I, H, 22)
    x = torch.randn(M, H, generator=torch.Generator().manual_seed(23))
    pushes = [(5, "add", [1.0, -1.0, 2.0]), (None, "mul", [1.0, 0.5, 2.0])]
    ref = omlp.swiglu_push(omlp.q8_linear(x, Wg, sg), omlp.q8_linear(x, Wu, su), pushes, T=1)
    Wi = torch.stack([Wg, Wu], dim=1).reshape(2 * I, H)
    si = torch.stack([sg, su], dim=1).reshape(2 * I, H // 128)
    announce(f"gemv g128 swiglu I{I}")
    a = ops.gemv(x.to(dev), Wi.to(dev), si.to(dev), epilogue="swiglu", pushes=ops.pack_pushes(pushes, dev))
    torch.cuda.synchronize()
    assert oracle.rel_err(a.cpu(), ref) <= TOL


@pytest.mark.parametrize("gs", [True, False])
@pytest.mark.parametrize("M,N,K", [(3, 1024, 3584), (1, 1024, 2048), (8, 1000, 2048), (3, 4096, 1024)])
def test_gemv_fixed_order_accumulate_is_repeatable(gs, M, N, K):
    """The "add_fixed" epilogue (every output summed in one order: 4-row blocks over all of K where the split-K form
    would split) agrees with the oracle's int8 product and with the split "add" form to fp32 rounding, and two calls
    from the same residual give bitwise the same result."""
    dev = device()
    g = torch.Generator().manual_seed(N + K + M)
    w = torch.randn(N, K, generator=g) * 0.02
    W, s = omlp.q8_quantize(w) if gs else _weights(N, K, torch.int8, seed=N + K)
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(M)) * 2.0
    base = torch.randn(M, N, generator=torch.Generator().manual_seed(9))
    ref = base + omlp.q8_linear(x, W, s)
    announce(f"gemv add_fixed M{M} N{N} K{K} gs {gs}")
    Wd, sd, xd = W.to(dev), s.to(dev), x.to(dev)
    outs = []
    for epi in ("add_fixed", "add_fixed", "add"):
        acc = base.to(dev)
        ops.gemv(xd, Wd, sd, out=acc, epilogue=epi)
        outs.append(acc)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
    assert oracle.rel_err(outs[0].cpu(), ref) <= TOL
    assert oracle.rel_err(outs[2].cpu(), outs[0].cpu()) <= TOL


def test_gemv_gated_norm_fixed_order_is_repeatable():
    """The GDN output projection with its gated-norm prologue, "add_fixed" against "add" (rounding) and itself
    (bitwise)."""
    dev = device()
    M, K, N = 3, 2048, 1024
    g = torch.Generator().manual_seed(3)
    W, s = omlp.q8_quantize(torch.randn(N, K, generator=g) * 0.02)
    o = torch.randn(M, K, generator=g).to(dev)
    z = torch.randn(M, K, generator=g).to(dev)
    nw = (1.0 + 0.1 * torch.randn(128, generator=g)).to(dev)
    hs = torch.rand(K // 128, generator=g).to(dev)
    base = torch.randn(M, N, generator=g).to(dev)
    announce("gemv_gated_norm add_fixed")
    outs = []
    for epi in ("add_fixed", "add_fixed", "add"):
        acc = base.clone()
        ops.gemv_gated_norm(o, z, nw, W.to(dev), s.to(dev), acc, head_scale=hs, epilogue=epi)
        outs.append(acc)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
    assert oracle.rel_err(outs[2].cpu(), outs[0].cpu()) <= TOL


@pytest.mark.parametrize("M,N,K,epi", [(8, 7168, 1024, "swiglu"), (8, 1024, 2048, "add"), (8, 40008, 1024, "store"),
                                       (1, 40008, 1024, "store"), (1, 7168, 1024, "swiglu"), (5, 8224, 1024, "store")])
def test_gemv_group_scales_one_and_eight_rows(M, N, K, epi):
    """The decode GEMV at 1 and 8 rows of x (8 rows run tiles of 8 output rows) with the engine's q8 weights and the
    norm prologue: SwiGLU with pushes, the split-K accumulation, and the tile loop of a wide product (N 40008)."""
    dev = device()
    g = torch.Generator().manual_seed(N + M)
    W, s = omlp.q8_quantize(torch.randn(N, K, generator=g) * 0.02)
    x = torch.randn(M, K, generator=g) * 2.0
    nw = torch.randn(K, generator=g) * 0.1
    h = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-6) * (1.0 + nw)
    pushes = [(17, "add", [1.0, -1.0, 0.5]), (None, "mul", [0.5, 2.0, 1.5])] if epi == "swiglu" else []
    if epi == "swiglu":
        y = omlp.q8_linear(h, W, s)
        ref = omlp.swiglu_push(y[:, 0::2], y[:, 1::2], pushes, T=1)
    else:
        ref = omlp.q8_linear(h, W, s)
    base = torch.randn(M, N, generator=g) if epi == "add" else None
    announce(f"gemv g128 M{M} N{N} K{K} {epi}")
    out = base.to(dev) if base is not None else None
    y = ops.gemv(x.to(dev), W.to(dev), s.to(dev), out=out, epilogue=epi,
                 pushes=ops.pack_pushes(pushes, dev) if pushes else None, prenorm=(None, nw.to(dev), 1e-6, None))
    torch.cuda.synchronize()
    got = y.cpu() - base if base is not None else y.cpu()
    e = oracle.rel_err(got, ref)
    print(f"gemv M{M} N{N} {epi}: rel err {e:.2e}")
    assert e <= TOL
