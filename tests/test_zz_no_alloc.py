"""The allocation-free attention decode entry point (q35_gated_attn_decode_noalloc) against the workspace entry point
it mirrors (q35_gated_attn_decode), through the C ABI: bitwise equal outputs on two calls in a row, the second with
a smaller input, and a host-side rejection of a request beyond its fixed scratch."""
import ctypes

import pytest
import torch

import q35hip
from q35hip import _lib, workloads
from gpu_util import announce, device

pytestmark = pytest.mark.gpu


def _call(L, d, out, cos, sin, noalloc):
    B, Hq, D = d["q"].shape
    Hkv, max_len = d["k_cache"].shape[1], d["k_cache"].shape[2]
    stream = torch.cuda.current_stream().cuda_stream
    args = [d["q"].data_ptr(), d["k_cache"].data_ptr(), d["v_cache"].data_ptr(), d["gate"].data_ptr(),
            d["cache_len"].data_ptr(), cos.data_ptr(), sin.data_ptr(), out.data_ptr(), _lib.Q35_F32,
            B, Hq, Hkv, D, max_len, 2 * cos.shape[1], ctypes.c_float(D ** -0.5), 0]
    if noalloc:
        return L.q35_gated_attn_decode_noalloc(*args, stream)
    ws = torch.empty(L.q35_gated_attn_decode_workspace_bytes(B, Hq, Hkv, D, max_len, 0), dtype=torch.uint8,
                     device=out.device)
    return L.q35_gated_attn_decode(*args, ws.data_ptr(), ws.numel(), stream)


def test_noalloc_decode_matches_workspace_entry_point():
    dev = device()
    L = q35hip.lib()
    assert L.q35_gated_attn_decode_noalloc_max_bytes() == 9 << 20
    for (B, N, max_len, seed) in ((32, 8192, 8192, 0), (3, 2300, 2312, 1)):
        lens = [N - 37 * r for r in range(B)]
        inp = workloads.to_device(workloads.attn_decode_inputs(B=B, N=N, max_len=max_len, seed=seed, lens=lens), dev)
        cos, sin = [t.to(dev) for t in workloads.rope_tables(max_len)]
        ref = torch.empty(B, 8 * 256, dtype=torch.float32, device=dev)
        got = torch.full_like(ref, float("nan"))
        announce(f"noalloc decode B{B} ctx{N} max_len {max_len}")
        assert _call(L, inp, ref, cos, sin, noalloc=False) == 0
        assert _call(L, inp, got, cos, sin, noalloc=True) == 0
        torch.cuda.synchronize()
        assert torch.equal(got, ref), f"B{B}: max diff {float((got - ref).abs().max())}"


def test_noalloc_decode_rejects_requests_beyond_its_scratch():
    L = q35hip.lib()
    fake = 0x1000
    need = L.q35_gated_attn_decode_workspace_bytes(512, 8, 2, 256, 8192, 0)
    assert need > L.q35_gated_attn_decode_noalloc_max_bytes()
    st = L.q35_gated_attn_decode_noalloc(fake, fake, fake, fake, fake, fake, fake, fake, _lib.Q35_F32, 512, 8, 2,
                                         256, 8192, 64, ctypes.c_float(0.0625), 0, None)
    assert st == _lib.Q35_ESCRATCH
    assert b"scratch" in L.q35_status_string(st)
