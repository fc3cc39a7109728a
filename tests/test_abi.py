"""The C ABI library loads and exports every entry point include/q35hip.h declares; argument validation rejects
bad calls before anything is launched (no GPU needed)."""
import ctypes
import os
import re

import pytest
import torch

import q35hip
from q35hip import _lib
from q35hip.build import LIB_PATH

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "q35hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(q35_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_boundary():
    names = declared_functions()
    for n in ["q35_gdn_recurrent", "q35_gdn_chunk_prefill", "q35_gated_attn_prefill", "q35_gated_attn_decode",
              "q35_resid_add_rows", "q35_gdn_conv", "q35_gdn_decode_fused", "q35_gated_rmsnorm", "q35_attn_prep",
              "q35_gemv",
              "q35_swiglu_push", "q35_add_rmsnorm", "q35_argmax_rows", "q35_gemv_norm"]:
        assert n in names


def test_library_built_and_exports_every_declared_symbol():
    assert os.path.exists(LIB_PATH), "libq35hip.so not built (run __graft_entry__.build())"
    raw = ctypes.CDLL(LIB_PATH)
    for n in declared_functions():
        assert hasattr(raw, n), f"{n} declared in q35hip.h but not exported"
    assert sorted(_lib.EXPORTS) == declared_functions()


def _c_kind(decl):
    """ctypes kind of one C declaration of the header (a parameter with its name, or a return type): P (any pointer
    or the stream handle), I64, I32, F32, SZ, or STR for a returned C string."""
    d = " ".join(decl.replace("const ", "").split())
    if d.startswith("char") and "*" in d:
        return "STR"
    if "*" in d or d.startswith("q35_stream_t"):
        return "P"
    return {"int64_t": "I64", "int": "I32", "float": "F32", "size_t": "SZ"}[d.split()[0]]


def test_bindings_match_the_header_prototypes():
    """Every prototype of include/q35hip.h has the parameter count and kinds, and the return kind, that the ctypes
    table of q35hip._lib binds (a wrong or missing argtype would pass garbage without any error)."""
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    protos = re.findall(r"([A-Za-z_][\w\s\*]*?)\b(q35_[a-z0-9_]+)\s*\(([^()]*)\)\s*;", text)
    kinds = {_lib.P: "P", _lib.I64: "I64", _lib.I32: "I32", _lib.F32: "F32", _lib.SZ: "SZ", ctypes.c_char_p: "STR"}
    seen = set()
    for ret, name, params in protos:
        seen.add(name)
        args, res = _lib._SIGS[name]
        plist = [] if params.strip() in ("", "void") else [x.strip() for x in params.split(",")]
        want = [_c_kind(x) for x in plist]
        got = [kinds[a] for a in args]
        assert got == want, f"{name}: ctypes {got} against the header's {want}"
        assert kinds[res] == _c_kind(ret.strip().split("\n")[-1]), f"{name}: return kind"
    assert seen == set(_lib._SIGS), sorted(seen ^ set(_lib._SIGS))


def test_status_strings_and_version():
    L = q35hip.lib()
    assert L.q35_abi_version() == 14
    assert L.q35_status_string(0) == b"ok"
    assert b"invalid" in L.q35_status_string(1)


def test_validation_rejects_without_launching():
    L = q35hip.lib()
    # null pointers
    assert L.q35_gdn_recurrent(None, None, None, None, None, None, None, None, 1, 1, 1, 1, 128, 128, 1, 1.0, 1,
                               None) == 1
    fake = 0x1000
    # unsupported head dim
    assert L.q35_gdn_recurrent(fake, fake, fake, fake, fake, None, fake, fake, 1, 1, 1, 1, 64, 64, 1, 1.0, 1,
                               None) == 2
    # value heads not a multiple of q/k heads
    assert L.q35_gdn_recurrent(fake, fake, fake, fake, fake, None, fake, fake, 1, 1, 3, 4, 128, 128, 1, 1.0, 1,
                               None) == 1
    # chunk size other than 64
    assert L.q35_gdn_chunk_workspace_bytes(1, 128, 16, 128, 128, 32, 1) == 0
    # the workspace follows the input dtype: bf16 pair records (128 positions) and fp32 chunk records (64)
    assert L.q35_gdn_chunk_workspace_bytes(1, 130, 2, 128, 128, 64, 1) == 2 * 2 * 131328
    assert L.q35_gdn_chunk_workspace_bytes(1, 130, 2, 128, 128, 64, 0) == 2 * 3 * 147712
    assert L.q35_gdn_chunk_workspace_bytes(1, 130, 2, 128, 128, 64, 2) == 0
    assert L.q35_gdn_chunk_prefill(fake, fake, fake, fake, fake, None, fake, fake, 1, 128, 16, 16, 128, 128, 1, 1.0,
                                   1, 32, fake, 1 << 30, None) == 2
    # workspace too small
    assert L.q35_gdn_chunk_prefill(fake, fake, fake, fake, fake, None, fake, fake, 1, 128, 16, 16, 128, 128, 1, 1.0,
                                   1, 64, fake, 16, None) == 3
    # attention: head dim 128 unsupported, GQA ratio 3 unsupported, odd rot invalid
    assert L.q35_gated_attn_prefill(fake, fake, fake, fake, fake, fake, 0, fake, 1, 16, 8, 2, 128, 64, 0.1,
                                    fake, 1 << 20, None) == 2
    assert L.q35_gated_attn_prefill(fake, fake, fake, fake, fake, fake, 0, fake, 1, 16, 6, 2, 256, 64, 0.1,
                                    fake, 1 << 20, None) == 2
    # prefill workspace: head dim other than 256 has none; too small a workspace is rejected
    assert L.q35_gated_attn_prefill_workspace_bytes(1, 100, 8, 2, 128) == 0
    assert L.q35_gated_attn_prefill_workspace_bytes(1, 100, 6, 2, 256) == 0
    # short sequence: rotated keys and transposed values only
    assert L.q35_gated_attn_prefill_workspace_bytes(1, 100, 8, 2, 256) == 2 * 2 * 128 * 256 * 2
    # T 4096: 128 query blocks, those with more than 32 key tiles (64 of them) split in two; per split block and
    # kv head, 2 halves x 4 waves x (32 x 256 + 128) fp32 partials
    kv = 2 * 2 * 4096 * 256 * 2
    parts = 64 * 2 * 2 * 4 * (8192 + 128) * 4
    assert L.q35_gated_attn_prefill_workspace_bytes(1, 4096, 8, 2, 256) == kv + parts
    assert L.q35_gated_attn_prefill(fake, fake, fake, fake, fake, fake, 0, fake, 1, 100, 8, 2, 256, 64, 0.1,
                                    fake, 16, None) == 3
    assert L.q35_gated_attn_decode(fake, fake, fake, fake, fake, fake, fake, fake, 1, 1, 8, 2, 256, 128, 63, 0.1,
                                   0, fake, 1 << 20, None) == 1
    assert L.q35_gated_attn_decode(fake, fake, fake, fake, fake, fake, fake, fake, 1, 1, 8, 2, 256, 128, 64, 0.1,
                                   0, fake, 8, None) == 3
    assert L.q35_gated_attn_decode(fake, fake, fake, fake, fake, fake, fake, fake, 2, 1, 8, 2, 256, 128, 64, 0.1,
                                   0, fake, 1 << 20, None) == 2
    assert L.q35_resid_add_rows(None, fake, None, 1, 1, 8, 1, 0, None) == 1
    # front-end kernels: null pointers, inconsistent widths, unsupported sizes
    assert L.q35_gdn_conv(None, 6144, fake, None, fake, fake, fake, 0, 0, fake, fake, fake, fake, fake, 1, 1, 16,
                          128, 16, 128, 4, 0, None) == 1
    assert L.q35_gdn_conv(fake, 100, fake, None, fake, fake, fake, 0, 0, fake, fake, fake, fake, fake, 1, 1, 16, 128,
                          16, 128, 4, 0, None) == 1
    assert L.q35_gdn_conv(fake, 6176, fake, None, fake, fake, fake, 6144, 6160, fake, fake, fake, fake, fake, 1, 1,
                          16, 128, 16, 128, 9, 0, None) == 2
    assert L.q35_gated_rmsnorm(fake, fake, 2048, fake, None, fake, 4, 16, 64, 1e-6, 0, None) == 2
    # fused GDN decode step: null pointers, a z window past the row, d != 128 (H 16, d 128: C 6144, ldy 8224)
    assert L.q35_gdn_decode_fused(None, 8224, fake, None, fake, fake, fake, 8192, 8208, 6144, fake, fake, None, 1e-6,
                                  0.088, fake, 1, 16, 128, 4, None) == 1
    assert L.q35_gdn_decode_fused(fake, 8224, fake, None, fake, fake, fake, 8192, 8208, 7000, fake, fake, None, 1e-6,
                                  0.088, fake, 1, 16, 128, 4, None) == 1
    assert L.q35_gdn_decode_fused(fake, 4128, fake, None, fake, fake, fake, 4096, 4112, 3072, fake, fake, None, 1e-6,
                                  0.125, fake, 1, 16, 64, 4, None) == 2
    assert L.q35_gated_rmsnorm(fake, fake, 100, fake, None, fake, 4, 16, 128, 1e-6, 0, None) == 1
    assert L.q35_attn_prep(fake, 5120, fake, fake, 1e-6, fake, fake, 64, None, fake, fake, None, None, fake, fake, 16,
                           1, 1, 8, 2, 256, None) == 1
    assert L.q35_attn_prep(fake, 5120, fake, fake, 1e-6, fake, fake, 60, fake, fake, fake, None, None, fake, fake,
                           16, 1, 1, 8, 2, 256, None) == 2
    # decode GEMV: K not a multiple of 256, too many rows, odd N for the SwiGLU epilogue, unknown weight type
    assert L.q35_gemv(fake, 1000, fake, 2, fake, fake, 64, 3, 64, 1000, 0, None, 0, 1, None, 0, 0, None) == 2
    assert L.q35_gemv(fake, 1024, fake, 2, fake, fake, 64, 9, 64, 1024, 0, None, 0, 1, None, 0, 0, None) == 2
    assert L.q35_gemv(fake, 1024, fake, 2, fake, fake, 64, 3, 63, 1024, 2, None, 0, 1, None, 0, 0, None) == 1
    assert L.q35_gemv(fake, 1024, fake, 1, fake, fake, 64, 3, 64, 1024, 0, None, 0, 1, None, 0, 0, None) == 2
    # group-128 int8 weights need their scales
    assert L.q35_gemv(fake, 1024, fake, 3, None, fake, 64, 3, 64, 1024, 0, None, 0, 1, None, 0, 0, None) == 1
    # prefill GEMM: weight formats other than int8, group scales over K not a multiple of 128, no scales
    assert L.q35_gemm_q8(fake, 1024, fake, 1, fake, fake, 64, 100, 64, 1024, 0, None, 0, 1, None, 0, 0, None) == 2
    assert L.q35_gemm_q8(fake, 192, fake, 3, fake, fake, 64, 100, 64, 192, 0, None, 0, 1, None, 0, 0, None) == 2
    assert L.q35_gemm_q8(fake, 1024, fake, 3, None, fake, 64, 100, 64, 1024, 0, None, 0, 1, None, 0, 0, None) == 1
    assert L.q35_swiglu_push(fake, fake, 3, 64, None, 2, 1, None, 0, 0, None) == 1
    assert L.q35_add_rmsnorm(fake, 1024, None, 0, fake, fake, 1024, 3, 1022, 1e-6, None) == 2
    assert L.q35_add_rmsnorm(fake, 512, None, 0, fake, fake, 1024, 3, 1024, 1e-6, None) == 1
    # split forms: the norm's split output needs H a multiple of 8; the split GEMM validates as q35_gemm_q8
    assert L.q35_add_rmsnorm_split(fake, 1028, None, 0, fake, fake, 1028, 3, 1028, 1e-6, None) == 2
    assert L.q35_gemm_q8_split(fake, 192, fake, 3, fake, fake, 64, 100, 64, 192, 0, None, 0, 1, None, 0, 0, None) == 2
    assert L.q35_gemm_q8_split(None, 1024, fake, 3, fake, fake, 64, 100, 64, 1024, 0, None, 0, 1, None, 0, 0, None) == 1
    # SwiGLU with split output (epilogue 3): N / 2 must be a multiple of 8; epilogue 4 does not exist
    assert L.q35_gemm_q8(fake, 1024, fake, 3, fake, fake, 64, 100, 36, 1024, 3, None, 0, 1, None, 0, 0, None) == 2
    assert L.q35_gemm_q8(fake, 1024, fake, 3, fake, fake, 64, 100, 64, 1024, 4, None, 0, 1, None, 0, 0, None) == 1
    assert L.q35_gated_rmsnorm_split(fake, fake, 2048, fake, None, fake, 3, 16, 64, 1e-6, None) == 2
    # activation capture: only with the SwiGLU epilogues, neuron strides of at least N / 2, 4-byte aligned
    assert L.q35_gemv(fake, 1024, fake, 2, fake, fake, 64, 3, 64, 1024, 0, None, 0, 1, fake, 64, 64, None) == 1
    assert L.q35_gemv(fake, 1024, fake, 2, fake, fake, 64, 3, 64, 1024, 5, None, 0, 1, None, 0, 0, None) == 1
    assert L.q35_gemv(fake, 1024, fake, 2, fake, fake, 64, 3, 64, 1024, 2, None, 0, 1, fake, 31, 64, None) == 1
    assert L.q35_gemm_q8(fake, 1024, fake, 3, fake, fake, 64, 100, 64, 1024, 1, None, 0, 1, fake, 64, 64, None) == 1
    assert L.q35_gemm_q8(fake, 1024, fake, 3, fake, fake, 64, 100, 64, 1024, 2, None, 0, 1, fake, 32, 31, None) == 1
    assert L.q35_gemm_q8(fake, 1024, fake, 3, fake, fake, 64, 100, 64, 1024, 3, None, 0, 1, fake + 2, 32, 32,
                         None) == 1
    assert L.q35_swiglu_push(fake, fake, 3, 64, None, 0, 1, fake, 63, 64, None) == 1
    # argmax: ld shorter than the row, no rows
    assert L.q35_argmax_rows(fake, 100, 3, 101, fake, None, None) == 1
    assert L.q35_argmax_rows(fake, 100, 0, 100, fake, None, None) == 1
    # gemv_norm: no norm weight; x_out overlapping x (the other blocks would read it while it is written)
    assert L.q35_gemv_norm(fake, None, None, 1024, None, 1e-6, fake, 2, fake, fake, 64, 3, 64, 1024, 0, None, 0, 1,
                           None, 0, 0, None) == 1
    assert L.q35_gemv_norm(fake, None, fake, 1024, fake, 1e-6, fake, 2, fake, fake, 64, 3, 64, 1024, 0, None, 0, 1,
                           None, 0, 0, None) == 1


def test_decode_workspace_scales_with_splits():
    """The workspace holds one partial per split; a split request is rounded to a power-of-two span of at most
    1024 keys (64 keys x 16 tiles), so 8 and 16 splits of 8192 keys are honoured and 4 becomes 8."""
    L = q35hip.lib()
    a = L.q35_gated_attn_decode_workspace_bytes(3, 8, 2, 256, 8192, 8)
    b = L.q35_gated_attn_decode_workspace_bytes(3, 8, 2, 256, 8192, 16)
    c = L.q35_gated_attn_decode_workspace_bytes(3, 8, 2, 256, 8192, 4)
    assert a > 0 and b == 2 * a and c == a


def test_no_kernel_spills_registers_or_uses_scratch():
    """Every gfx950 kernel of the built library (read from its code objects' metadata) keeps its values in registers:
    no VGPR spills and no private (scratch) segment, in particular the decode GEMV at 1 and 8 rows of x. (SGPR spills
    go to VGPR lanes, not to memory, and are allowed.)"""
    from kernel_meta import kernel_metadata
    md = kernel_metadata(LIB_PATH)
    assert len(md) > 100
    assert any("gemv_kernelIaLi1E" in k["name"] for k in md) and any("gemv_kernelIaLi8E" in k["name"] for k in md)
    bad = [(k["name"], k.get(".vgpr_spill_count"), k.get(".private_segment_fixed_size"))
           for k in md if k.get(".vgpr_spill_count", 0) or k.get(".private_segment_fixed_size", 0)]
    assert not bad, bad[:5]


def test_noalloc_scratch_capacity_boundary():
    """The allocation-free decode's fixed scratch (9 MiB) holds the partials of B <= 142 rows at an 8192-token cache
    (Hq 8, Hkv 2, D 256, default splits) and not of 143: host-side sizes only."""
    L = q35hip.lib()
    cap = L.q35_gated_attn_decode_noalloc_max_bytes()
    assert cap == 9 << 20
    assert L.q35_gated_attn_decode_workspace_bytes(128, 8, 2, 256, 8192, 0) <= cap
    assert L.q35_gated_attn_decode_workspace_bytes(142, 8, 2, 256, 8192, 0) <= cap
    assert L.q35_gated_attn_decode_workspace_bytes(143, 8, 2, 256, 8192, 0) > cap


def test_ops_refuse_cpu_tensors():
    x = torch.zeros(1, 4, 16, 128)
    g = torch.zeros(1, 4, 16)
    with pytest.raises(Exception, match="no CPU|HIP device"):
        q35hip.chunk_gated_delta_rule(x, x, x, g, g)
    with pytest.raises(Exception, match="no CPU|HIP device"):
        q35hip.recurrent_gated_delta_rule(x, x, x, g, g, None, True)


def test_fused_gdn_step_and_fp32_decode_refuse_cpu_tensors():
    """The fused GDN decode step and the fp32-output attention decode have no CPU path either."""
    B, H, d, K = 1, 2, 128, 4
    C = 3 * H * d
    y = torch.zeros(B, C + H * d + 2 * H)
    with pytest.raises(Exception, match="no CPU|HIP device"):
        q35hip.ops.gdn_decode_fused_(y, torch.zeros(C, 1, K), torch.zeros(B, K - 1, C), torch.zeros(H), torch.zeros(H),
                                     torch.zeros(B, H, d, d), torch.ones(d), b_off=C + H * d, a_off=C + H * d + H,
                                     z_off=C)
    q = torch.zeros(1, 8, 256, dtype=torch.bfloat16)
    kc = torch.zeros(1, 2, 64, 256, dtype=torch.bfloat16)
    with pytest.raises(Exception, match="no CPU|HIP device"):
        q35hip.ops.gated_attention_decode(q, kc, kc, torch.zeros(1, 2048, dtype=torch.bfloat16),
                                          torch.ones(1, dtype=torch.int32), torch.zeros(64, 32), torch.zeros(64, 32),
                                          out_dtype=torch.float32)


def test_decode_from_projection_rejects_without_launching():
    """q35_gated_attn_decode_proj refuses bad arguments before any HIP call (Hq 8, Hkv 2, D 256: y rows of 5120
    floats), and its torch op has no CPU path."""
    L = q35hip.lib()
    fake = 0x1000
    W = 8 * 2 * 256 + 2 * 2 * 256

    def call(y=fake, ldy=W, qnw=fake, knw=fake, Hq=8, Hkv=2, D=256, ws_bytes=1 << 20):
        return L.q35_gated_attn_decode_proj(y, ldy, qnw, knw, 1e-6, fake, fake, fake, fake, fake, fake, 1, 1, Hq, Hkv,
                                            D, 128, 64, 0.0625, 0, fake, ws_bytes, None)
    assert call(y=None) == 1                 # null y
    assert call(knw=None) == 1               # null norm weight
    assert call(ldy=W - 4) == 1              # rows too short for [q | gate] x Hq, k, v
    assert call(y=fake + 4) == 2             # y not 16-byte aligned
    assert call(ldy=W + 2) == 2              # row stride not a multiple of 4 floats
    assert call(Hq=6) == 2                   # 3 query heads per kv head
    assert call(D=128, ldy=8 * 256 + 4 * 128) == 2  # head dim other than 256
    assert call(ws_bytes=8) == 3             # workspace too small
    y = torch.zeros(1, W)
    kc = torch.zeros(1, 2, 64, 256, dtype=torch.bfloat16)
    with pytest.raises(Exception, match="no CPU|HIP device"):
        q35hip.ops.gated_attention_decode_proj(y, torch.zeros(256), torch.zeros(256), kc, kc.clone(),
                                               torch.zeros(1, dtype=torch.int32), torch.zeros(64, 32),
                                               torch.zeros(64, 32), num_heads=8)


def test_prefill_from_projection_rejects_without_launching():
    """q35_gated_attn_prefill_proj refuses bad arguments before any HIP call (Hq 8, Hkv 2, D 256, T 130 tokens at
    pos0 0 into a 192-row cache: y rows of 5120 floats); its workspace is the own-keys prefill's plus the rotated
    queries, and its torch op has no CPU path."""
    L = q35hip.lib()
    fake = 0x1000
    W = 8 * 2 * 256 + 2 * 2 * 256

    def call(y=fake, ldy=W, qnw=fake, knw=fake, pos0=0, T=130, Hq=8, Hkv=2, D=256, max_len=192, rot=64,
             ws_bytes=1 << 24):
        return L.q35_gated_attn_prefill_proj(y, ldy, qnw, knw, 1e-6, fake, fake, pos0, fake, fake, fake, 1, T, Hq, Hkv,
                                             D, max_len, rot, 0.0625, fake, ws_bytes, None)
    assert call(y=None) == 1                 # null y
    assert call(knw=None) == 1               # null norm weight
    assert call(ldy=W - 4) == 1              # rows too short for [q | gate] x Hq, k, v
    assert call(pos0=63) == 1                # positions 63 .. 192 run past the cache
    assert call(pos0=-1) == 1
    assert call(T=0) == 1
    assert call(y=fake + 4) == 2             # y not 16-byte aligned
    assert call(ldy=W + 2) == 2              # row stride not a multiple of 4 floats
    assert call(Hq=6) == 2                   # 3 query heads per kv head
    assert call(D=128, ldy=8 * 256 + 4 * 128) == 2  # head dim other than 256
    assert call(rot=24) == 2                 # rotary dims not a multiple of 16
    assert call(ws_bytes=8) == 3             # workspace too small
    # 2 x [1, 2, 192, 256] bf16 (keys, values^T), then [1, 130, 8, 256] bf16 rotated queries; no split blocks
    plain = L.q35_gated_attn_prefill_workspace_bytes(1, 130, 8, 2, 256)
    assert plain == 2 * 2 * 192 * 256 * 2
    assert L.q35_gated_attn_prefill_proj_workspace_bytes(1, 130, 8, 2, 256) == plain + 130 * 8 * 256 * 2
    assert L.q35_gated_attn_prefill_proj_workspace_bytes(1, 130, 6, 2, 256) == 0
    assert call(ws_bytes=plain + 130 * 8 * 256 * 2 - 256) == 3
    y = torch.zeros(1, 4, W)
    kc = torch.zeros(1, 2, 64, 256, dtype=torch.bfloat16)
    with pytest.raises(Exception, match="no CPU|HIP device"):
        q35hip.ops.gated_attention_prefill_proj(y, torch.zeros(256), torch.zeros(256), kc, kc.clone(),
                                                torch.zeros(64, 32), torch.zeros(64, 32), num_heads=8)


def test_gemv_norm_argmax_rejects_without_launching():
    """q35_gemv_norm_argmax refuses bad arguments before any HIP call (3 rows, N 151936, K 1024, int8 weights with
    group scales), and its torch op has no CPU path."""
    L = q35hip.lib()
    fake = 0x1000

    def call(slots=fake, idx=fake, M=3, K=1024, nw=fake):
        return L.q35_gemv_norm_argmax(fake, None, None, K, nw, 1e-6, fake, 3, fake, fake, 151936, M, 151936, K, slots,
                                      idx, None)
    assert call(slots=None) == 1             # no argmax slots
    assert call(idx=None) == 1               # no index output
    assert call(nw=None) == 1                # no norm weight
    assert call(slots=fake + 4) == 2         # slots not 8-byte aligned
    assert call(M=9) == 2                    # more rows than the GEMV takes
    assert call(K=1000) == 2                 # K not a multiple of 256
    x = torch.zeros(3, 1024)
    with pytest.raises(Exception, match="no CPU|HIP device"):
        q35hip.ops.gemv_norm_argmax(x, torch.zeros(8, 1024, dtype=torch.int8), torch.ones(8, 8),
                                    (None, torch.zeros(1024), 1e-6, None), torch.zeros(3, dtype=torch.int64))


def test_prefill_over_cache_from_projection_rejects_without_launching():
    """q35_gated_attn_prefill_cached_proj refuses bad arguments before any HIP call (Hq 8, Hkv 2, D 256, T 100 over a
    448-row cache); its workspace is V^T of the cache plus the rotated queries, and its torch op has no CPU path."""
    L = q35hip.lib()
    fake = 0x1000
    W = 8 * 2 * 256 + 2 * 2 * 256

    def call(y=fake, ldy=W, pos=fake, T=100, Hq=8, D=256, max_len=448, rot=64, ws_bytes=1 << 24):
        return L.q35_gated_attn_prefill_cached_proj(y, ldy, fake, fake, 1e-6, fake, fake, pos, fake, fake, fake, 1, T,
                                                    Hq, 2, D, max_len, rot, 0.0625, fake, ws_bytes, None)
    assert call(y=None) == 1                 # null y
    assert call(pos=None) == 1               # null positions
    assert call(ldy=W - 4) == 1              # rows too short for [q | gate] x Hq, k, v
    assert call(T=449) == 1                  # more tokens than the cache holds
    assert call(y=fake + 4) == 2             # y not 16-byte aligned
    assert call(max_len=450, T=100) == 2     # cache length not a multiple of 64
    assert call(Hq=6) == 2                   # 3 query heads per kv head
    assert call(rot=24) == 2                 # rotary dims not a multiple of 16
    assert call(ws_bytes=8) == 3             # workspace too small
    need = 2 * 256 * 448 * 2 + 100 * 8 * 256 * 2
    assert L.q35_gated_attn_prefill_cached_proj_workspace_bytes(1, 100, 8, 2, 256, 448) == need
    assert L.q35_gated_attn_prefill_cached_proj_workspace_bytes(1, 100, 8, 2, 256, 450) == 0
    assert call(ws_bytes=need - 256) == 3
    y = torch.zeros(1, 4, W)
    kc = torch.zeros(1, 2, 64, 256, dtype=torch.bfloat16)
    with pytest.raises(Exception, match="no CPU|HIP device"):
        q35hip.ops.gated_attention_prefill_cached_proj(y, torch.zeros(256), torch.zeros(256), kc, kc.clone(),
                                                       torch.zeros(1, dtype=torch.int32), torch.zeros(64, 32),
                                                       torch.zeros(64, 32), num_heads=8)


def test_split_activation_layout():
    """The int8 GEMM's split layout (ops.split_activations, which the norm's split output and the split GEMM follow):
    per row, each group of 8 inputs is 32 bytes, the 8 bf16 hi parts then the 8 bf16 lo parts; hi is x rounded to
    bf16 (nearest even), hi + lo recovers x to 2^-16 relative (lo is the rounded remainder), exactly when x has at
    most 16 significant bits."""
    from q35hip import ops
    g = torch.Generator().manual_seed(5)
    x = torch.randn(3, 40, generator=g) * torch.logspace(-3, 3, 40)
    w = ops.split_activations(x)
    assert w.dtype == torch.int32 and w.shape == x.shape
    parts = w.view(torch.bfloat16).view(3, 5, 16)
    hi, lo = parts[..., :8].reshape(3, 40), parts[..., 8:].reshape(3, 40)
    assert torch.equal(hi, x.to(torch.bfloat16))
    assert torch.equal(lo, (x - hi.float()).to(torch.bfloat16))
    assert bool(((hi.float() + lo.float() - x).abs() <= x.abs() * 2.0 ** -16).all())
    exact = torch.tensor([[1.0, -3.0, 0.5, 1 + 2.0 ** -10, 0.0, 1024.0, -2.0 ** -20, 3 * 2.0 ** -9]])
    e = ops.split_activations(exact).view(torch.bfloat16).view(1, 1, 16)
    assert torch.equal(e[..., :8].float() + e[..., 8:].float(), exact.view(1, 1, 8))
    # a planted layout mistake (hi and lo interleaved per value) reads back as different words
    wrong = torch.stack([x.to(torch.bfloat16), (x - hi.float()).to(torch.bfloat16)], -1).reshape(3, 80)
    assert not torch.equal(wrong.view(torch.int32), w)
    with pytest.raises(ValueError):
        ops.split_activations(torch.zeros(2, 12))

