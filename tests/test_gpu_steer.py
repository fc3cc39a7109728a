"""Residual steering add on the GPU: bitwise equal to the oracle (fp32 and bf16 residual streams)."""
import pytest
import torch

import oracle
import q35hip
from gpu_util import announce, device

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("T", [1, 7, 2048])
def test_steer_rows_plus_none_minus(dtype, T):
    dev = device()
    gen = torch.Generator().manual_seed(T)
    x = torch.randn(3, T, 1024, generator=gen).to(dtype)
    v = torch.randn(1024, generator=gen)
    vecs = torch.stack([v, -v])
    rows = torch.tensor([0, -1, 1], dtype=torch.int32)  # +v, none, -v
    ref = oracle.residual_steer_add(x, vecs, rows)
    xd = x.to(dev)
    announce(f"steer add T{T} {dtype}")
    q35hip.residual_steer_add_(xd, vecs.to(dev), rows.to(dev))
    assert torch.equal(xd.cpu(), ref)


def test_steer_default_row_clamp():
    """vec_of_row None: row r uses vector min(r, nvec - 1), as the WGSL resAdd clamps to 3."""
    dev = device()
    x = torch.randn(6, 5, 1000)
    vecs = torch.randn(4, 1000)
    ref = oracle.residual_steer_add(x, vecs, None)
    xd = x.to(dev)
    q35hip.residual_steer_add_(xd, vecs.to(dev), None)
    assert torch.equal(xd.cpu(), ref)
