"""The int8 prefill GEMM (q35_gemm_q8) on the GPU against the oracle's int8 product (oracle.mlp.q8_linear, fp32 on
the dequantised weights) and the oracle's SwiGLU + push semantics. The GEMM computes bf16 MFMA products on a hi + lo
split of x, so it agrees with the fp32 product to about 1e-5 (tolerance 1e-4 here)."""
import pytest
import torch

import oracle
from oracle import mlp as omlp
from q35hip import ops
from gpu_util import announce, device

pytestmark = pytest.mark.gpu
TOL = 1e-4


def _q8(N, K, seed):
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(N, K, generator=g) * 0.02
    s = w.abs().amax(dim=1) / 127.0
    q = torch.clamp(torch.round(w / s[:, None]), -127, 127).to(torch.int8)
    return q, s


# shapes: the stack's projections at small M, ragged M and N (masked edges), M past the 128-row tile threshold
@pytest.mark.parametrize("M,N,K", [(9, 8224, 1024), (100, 1024, 2048), (300, 130, 64), (2048, 5120, 1024),
                                   (1500, 1024, 3584)])
def test_gemm_q8_store_and_accumulate(M, N, K):
    dev = device()
    q, s = _q8(N, K, M + N)
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(K)) * 3.0
    ref = omlp.q8_linear(x, q, s)
    announce(f"gemm_q8 store M{M} N{N} K{K}")
    y = ops.gemm_q8(x.to(dev), q.to(dev), s.to(dev))
    e = oracle.rel_err(y.cpu(), ref)
    print(f"gemm_q8 M{M} N{N} K{K}: rel err {e:.2e}")
    assert e <= TOL
    base = torch.randn(M, N)
    out = base.to(dev)
    ops.gemm_q8(x.to(dev), q.to(dev), s.to(dev), out=out, epilogue="add")
    assert oracle.rel_err(out.cpu() - base, ref) <= TOL


def test_gemm_q8_strided_rows_of_x():
    """x rows with a leading dimension past K (a column slice of a wider buffer)."""
    dev = device()
    q, s = _q8(256, 128, 3)
    wide = torch.randn(70, 200, generator=torch.Generator().manual_seed(4))
    ref = omlp.q8_linear(wide[:, :128], q, s)
    announce("gemm_q8 strided x")
    y = ops.gemm_q8(wide.to(dev)[:, :128], q.to(dev), s.to(dev))
    assert oracle.rel_err(y.cpu(), ref) <= TOL


@pytest.mark.parametrize("M,T", [(40, 20), (2048, 2048), (6144, 2048)])
def test_gemm_q8_swiglu_with_pushes(M, T):
    """Interleaved (gate, up) rows, SwiGLU epilogue, pushes in order (add then mul on one neuron, an all-neuron add),
    push rows min(m / T, 3)."""
    dev = device()
    I, H = 3584, 1024
    qg, sg = _q8(I, H, 5)
    qu, su = _q8(I, H, 6)
    q = torch.stack([qg, qu], dim=1).reshape(2 * I, H).contiguous()
    s = torch.stack([sg, su], dim=1).reshape(2 * I).contiguous()
    x = torch.randn(M, H, generator=torch.Generator().manual_seed(M))
    pushes = [(7, "add", [1.0, 2.0, -1.0]), (7, "mul", [2.0, 0.5, 3.0]), (None, "add", [0.25, 0.0, -0.25])]
    ref = omlp.swiglu_push(omlp.q8_linear(x, qg, sg), omlp.q8_linear(x, qu, su), pushes, T=T)
    announce(f"gemm_q8 swiglu M{M} T{T}")
    a = ops.gemm_q8(x.to(dev), q.to(dev), s.to(dev), epilogue="swiglu", pushes=ops.pack_pushes(pushes, dev), T=T)
    e = oracle.rel_err(a.cpu(), ref)
    print(f"gemm_q8 swiglu M{M}: rel err {e:.2e}")
    assert e <= TOL


def _q8g(N, K, seed):
    """The engine's q8 format: one scale per group of 128 inputs of a row (oracle.mlp.q8_quantize)."""
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(N, K, generator=g) * 0.02 * (1.0 + 9.0 * (torch.arange(K) // 128 % 2))[None, :]
    return omlp.q8_quantize(w)


@pytest.mark.parametrize("M,N,K", [(9, 8224, 1024), (300, 130, 128), (2048, 5120, 1024), (1500, 1024, 3584),
                                   (6144, 1024, 2048), (6144, 8224, 1024)])
def test_gemm_q8_group_scales_store_and_accumulate(M, N, K):
    """Q35_I8_G128 weights (scales of neighbouring groups about a decade apart) against the oracle's per-group
    product: 64- and 128-row tiles of the register-staged kernel, the DMA-staged kernel, and at M 6144 N 8224 (the
    stack's GDN input projection) the DMA kernel on the first 8192 columns with the last 32 on the register-staged
    one."""
    dev = device()
    q, s = _q8g(N, K, M + N)
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(K)) * 3.0
    ref = omlp.q8_linear(x, q, s)
    announce(f"gemm_q8 g128 M{M} N{N} K{K}")
    y = ops.gemm_q8(x.to(dev), q.to(dev), s.to(dev))
    e = oracle.rel_err(y.cpu(), ref)
    print(f"gemm_q8 g128 M{M} N{N} K{K}: rel err {e:.2e}")
    assert e <= TOL
    base = torch.randn(M, N)
    out = base.to(dev)
    ops.gemm_q8(x.to(dev), q.to(dev), s.to(dev), out=out, epilogue="add")
    assert oracle.rel_err(out.cpu() - base, ref) <= TOL


def test_gemm_q8_group_scales_swiglu_with_pushes():
    dev = device()
    I, H, M, T = 3584, 1024, 2048, 2048
    qg, sg = _q8g(I, H, 31)
    qu, su = _q8g(I, H, 32)
    q = torch.stack([qg, qu], dim=1).reshape(2 * I, H).contiguous()
    s = torch.stack([sg, su], dim=1).reshape(2 * I, H // 128).contiguous()
    x = torch.randn(M, H, generator=torch.Generator().manual_seed(33))
    pushes = [(11, "mul", [2.0]), (None, "add", [0.5])]
    ref = omlp.swiglu_push(omlp.q8_linear(x, qg, sg), omlp.q8_linear(x, qu, su), pushes, T=T)
    announce("gemm_q8 g128 swiglu")
    a = ops.gemm_q8(x.to(dev), q.to(dev), s.to(dev), epilogue="swiglu", pushes=ops.pack_pushes(pushes, dev), T=T)
    assert oracle.rel_err(a.cpu(), ref) <= TOL


def test_gemm_q8_swiglu_placeholder_push_records():
    """Eight push records as the model passes them: real pushes on a few neurons (two on either side of a 128-neuron
    block boundary, one further on), the rest placeholders whose neuron index matches no neuron; batch rows of
    T = 200 tokens (push rows 0..2). Blocks that no record touches skip the push loop; the result equals the
    oracle's in-order pushes."""
    dev = device()
    I, H, M, T = 3584, 1024, 600, 200
    qg, sg = _q8g(I, H, 41)
    qu, su = _q8g(I, H, 42)
    q = torch.stack([qg, qu], dim=1).reshape(2 * I, H).contiguous()
    s = torch.stack([sg, su], dim=1).reshape(2 * I, H // 128).contiguous()
    x = torch.randn(M, H, generator=torch.Generator().manual_seed(43))
    none = (1 << 30, "add", [0.0])
    pushes = [(127, "add", [1.0, -2.0, 0.5]), none, (128, "mul", [2.0, 3.0, 0.5]), none, none,
              (3000, "add", [0.25, 0.5, 0.75]), none, (3000, "mul", [-1.0, 2.0, 1.5])]
    ref = omlp.swiglu_push(omlp.q8_linear(x, qg, sg), omlp.q8_linear(x, qu, su), pushes, T=T)
    announce("gemm_q8 g128 swiglu placeholder pushes")
    a = ops.gemm_q8(x.to(dev), q.to(dev), s.to(dev), epilogue="swiglu", pushes=ops.pack_pushes(pushes, dev), T=T)
    assert oracle.rel_err(a.cpu(), ref) <= TOL
    cols = [127, 128, 3000]  # the pushed neurons alone, at the GEMM's own error (an unapplied push would be O(1) off)
    assert oracle.rel_err(a.cpu()[:, cols], ref[:, cols]) <= TOL


@pytest.mark.parametrize("M,N,K,gs,epi", [(9, 8224, 1024, True, "store"), (300, 130, 128, False, "add"),
                                          (2048, 5120, 1024, True, "store"), (1500, 1024, 3584, True, "add"),
                                          (6144, 8224, 1024, True, "store"), (6144, 7168, 1024, True, "swiglu"),
                                          (2100, 4096, 512, False, "swiglu")])
def test_gemm_q8_split_input_equals_fp32_input(M, N, K, gs, epi):
    """x handed over already split (ops.split_activations: bf16 hi + lo per value, the GEMM's own split) gives the
    same product, bitwise, as fp32 x: both kernels (the DMA-staged one copies the split pieces straight into its
    fragment planes, the register-staged one stores them as loaded), with the DMA kernel's column and row tails
    (M 6144 N 8224; the SwiGLU rows past 45 panels at M 6144 N 7168) and ragged M, N."""
    dev = device()
    q, s = (_q8g if gs else _q8)(N, K, M + 7 * N)
    x = (torch.randn(M, K, generator=torch.Generator().manual_seed(M + K)) * 3.0).to(dev)
    qd, sd = q.to(dev), s.to(dev)
    pushes = None
    if epi == "swiglu":
        pushes = ops.pack_pushes([(5, "add", [1.0, -1.0, 2.0]), (None, "mul", [0.5, 2.0, 1.0])], dev)
    announce(f"gemm_q8 split input M{M} N{N} K{K} gs {gs} {epi}")
    xs = ops.split_activations(x)
    if epi == "add":
        base = torch.randn(M, N, generator=torch.Generator().manual_seed(1)).to(dev)
        a, b = base.clone(), base.clone()
        ops.gemm_q8(x, qd, sd, out=a, epilogue="add")
        ops.gemm_q8(xs, qd, sd, out=b, epilogue="add")
    else:
        a = ops.gemm_q8(x, qd, sd, epilogue=epi, pushes=pushes, T=max(1, M // 3))
        b = ops.gemm_q8(xs, qd, sd, epilogue=epi, pushes=pushes, T=max(1, M // 3))
    torch.cuda.synchronize()
    assert torch.equal(a, b), f"max diff {(a - b).abs().max().item():.3e}"


@pytest.mark.parametrize("M,N,K", [(6144, 7168, 1024), (300, 512, 256)])
def test_gemm_q8_swiglu_split_output(M, N, K):
    """The SwiGLU epilogue writing its output in the split layout (split_out, the down projection's input) equals
    ops.split_activations of the fp32 output bitwise, with pushes: the DMA kernel with its row tail (M 6144) and the
    register-staged kernel (N 512); down_proj on that output equals down_proj on the fp32 output bitwise."""
    dev = device()
    q, s = _q8g(N, K, 17 + M)
    x = (torch.randn(M, K, generator=torch.Generator().manual_seed(M)) * 2.0).to(dev)
    pushes = ops.pack_pushes([(3, "mul", [2.0, -1.0, 0.5]), (None, "add", [0.25, 0.0, -0.25])], dev)
    announce(f"gemm_q8 swiglu split output M{M} N{N} K{K}")
    a = ops.gemm_q8(x, q.to(dev), s.to(dev), epilogue="swiglu", pushes=pushes, T=max(1, M // 3))
    b = ops.gemm_q8(x, q.to(dev), s.to(dev), epilogue="swiglu", pushes=pushes, T=max(1, M // 3), split_out=True)
    torch.cuda.synchronize()
    assert b.dtype == torch.int32 and b.shape == a.shape
    assert torch.equal(b, ops.split_activations(a))
    qd, sd = _q8g(256, N // 2, 19)
    ya = ops.gemm_q8(a, qd.to(dev), sd.to(dev))
    yb = ops.gemm_q8(b, qd.to(dev), sd.to(dev))
    assert torch.equal(ya, yb)


@pytest.mark.parametrize("M,N,K", [(6144, 1024, 2048), (70, 300, 512), (2048, 4096, 1024)])
def test_gemm_q8_bf16_input_equals_fp32_input(M, N, K):
    """bf16 x (the attention output) gives bitwise the product of its fp32 values, store and accumulate, where the
    fp32 input also runs the register-staged kernel (N < 2048); at N 4096, K 1024 the fp32 input runs the DMA kernel
    (another K grouping) and the two agree to fp32 rounding (1e-5)."""
    dev = device()
    q, s = _q8g(N, K, 23 + M)
    xb = (torch.randn(M, K, generator=torch.Generator().manual_seed(M)) * 2.0).to(torch.bfloat16).to(dev)
    announce(f"gemm_q8 bf16 input M{M} N{N} K{K}")
    a = ops.gemm_q8(xb.float(), q.to(dev), s.to(dev))
    b = ops.gemm_q8(xb, q.to(dev), s.to(dev))
    base = torch.randn(M, N, generator=torch.Generator().manual_seed(2)).to(dev)
    c, d = base.clone(), base.clone()
    ops.gemm_q8(xb.float(), q.to(dev), s.to(dev), out=c, epilogue="add")
    ops.gemm_q8(xb, q.to(dev), s.to(dev), out=d, epilogue="add")
    torch.cuda.synchronize()
    if N < 2048:
        assert torch.equal(a, b) and torch.equal(c, d)
    else:
        assert oracle.rel_err(b.cpu(), a.cpu()) <= 1e-5 and oracle.rel_err(d.cpu(), c.cpu()) <= 1e-5

