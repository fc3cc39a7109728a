"""torch.library registration (namespace q35) of the HIP kernels, plus Python entry points whose signatures follow the
reference's replaceable functions.

Reference interfaces mirrored (HF: transformers 5.15.0 models/qwen3_5/modeling_qwen3_5.py, run by the reference's
tests/engine_ref.py):
  chunk_gated_delta_rule      <- torch_chunk_gated_delta_rule (HF:248-327, hub-kernel name "chunk_gated_delta_rule")
  recurrent_gated_delta_rule  <- torch_recurrent_gated_delta_rule (HF:330-380, "recurrent_gated_delta_rule")
  gated_attention_prefill     <- apply_rotary_pos_emb + eager_attention_forward + sigmoid gate (HF:656-698)
  gated_attention_decode      <- the same for one token over a KV cache (WGSL engine/kernels_qwen35.js:73-123)
  residual_steer_add_         <- layers[12] forward hook (tests/engine_ref.py:49-53), WGSL resAdd
                                 (engine/kernels.js:190-203)
Every op runs on the current HIP stream of its inputs' device; inputs are validated here (device, dtype, layout,
shape) and a bad call raises RuntimeError. CPU tensors raise: there is no CPU path in the product.
"""
import math

import torch

from . import _lib
from ._lib import Q35_BF16, Q35_F32, Q35_I8, Q35_I8_G128, Q35Error, check

_DT = {torch.float32: Q35_F32, torch.bfloat16: Q35_BF16}


def _ptr(t):
    return None if t is None else t.data_ptr()


def _stream(t):
    return torch.cuda.current_stream(t.device).cuda_stream


def _require(cond, msg):
    if not cond:
        raise Q35Error("q35hip: " + msg)


def _on_gpu(*ts):
    dev = None
    for t in ts:
        if t is None:
            continue
        _require(t.is_cuda, "inputs must be HIP device tensors (there is no CPU fallback)")
        _require(t.is_contiguous(), "inputs must be contiguous")
        dev = t.device if dev is None else dev
        _require(t.device == dev, "inputs must be on one device")


def _workspace(nbytes, device):
    return torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=device)


# ---------------------------------------------------------------- schema
_LIB = torch.library.Library("q35", "DEF")
_LIB.define("gdn_recurrent(Tensor q, Tensor k, Tensor v, Tensor g, Tensor beta, Tensor? initial_state, "
            "float scale, bool use_qk_l2norm) -> (Tensor, Tensor)")
_LIB.define("gdn_decode_step_(Tensor q, Tensor k, Tensor v, Tensor g, Tensor beta, Tensor(a!) state, "
            "float scale, bool use_qk_l2norm) -> Tensor")
_LIB.define("gdn_chunk_prefill(Tensor q, Tensor k, Tensor v, Tensor g, Tensor beta, Tensor? initial_state, "
            "int chunk_size, float scale, bool use_qk_l2norm) -> (Tensor, Tensor)")
_LIB.define("gated_attn_prefill(Tensor q, Tensor k, Tensor v, Tensor gate, Tensor cos, Tensor sin, int pos0, "
            "float scale) -> Tensor")
_LIB.define("gated_attn_prefill_cached(Tensor q, Tensor k_cache, Tensor v_cache, Tensor gate, Tensor pos, "
            "Tensor cos, Tensor sin, float scale) -> Tensor")
_LIB.define("gated_attn_decode(Tensor q, Tensor k_cache, Tensor v_cache, Tensor gate, Tensor cache_len, "
            "Tensor cos, Tensor sin, float scale, int splits, bool f32_out=False) -> Tensor")
_LIB.define("gated_attn_decode_proj(Tensor y, Tensor q_norm_w, Tensor k_norm_w, float eps, Tensor(a!) k_cache, "
            "Tensor(b!) v_cache, Tensor pos, Tensor cos, Tensor sin, int Hq, float scale, int splits, "
            "bool f32_out=False) -> Tensor")
_LIB.define("gated_attn_prefill_proj(Tensor y, Tensor q_norm_w, Tensor k_norm_w, float eps, Tensor(a!) k_cache, "
            "Tensor(b!) v_cache, int pos0, Tensor cos, Tensor sin, int Hq, float scale) -> Tensor")
_LIB.define("gated_attn_prefill_cached_proj(Tensor y, Tensor q_norm_w, Tensor k_norm_w, float eps, "
            "Tensor(a!) k_cache, Tensor(b!) v_cache, Tensor pos, Tensor cos, Tensor sin, int Hq, "
            "float scale) -> Tensor")
_LIB.define("resid_add_rows_(Tensor(a!) x, Tensor vecs, Tensor? vec_of_row) -> ()")
_LIB.define("gdn_conv(Tensor y, Tensor conv_w, Tensor? conv_bias, Tensor(a!) conv_state, Tensor A_log, "
            "Tensor dt_bias, int b_off, int a_off, int Hk, int dk, int Hv, int dv, bool bf16_out) "
            "-> (Tensor, Tensor, Tensor, Tensor, Tensor)")
_LIB.define("gated_rmsnorm(Tensor o, Tensor z, Tensor w, Tensor? head_scale, float eps) -> Tensor")
_LIB.define("gated_rmsnorm_split(Tensor o, Tensor z, Tensor w, Tensor? head_scale, float eps) -> Tensor")
_LIB.define("gdn_decode_fused_(Tensor y, Tensor conv_w, Tensor? conv_bias, Tensor(a!) conv_state, Tensor A_log, "
            "Tensor dt_bias, int b_off, int a_off, int z_off, Tensor(b!) state, Tensor norm_w, Tensor? head_scale, "
            "float eps, float scale) -> Tensor")
_LIB.define("gemv_(Tensor x, Tensor W, Tensor? w_scale, Tensor(a!) y, int epilogue, Tensor? pushes, int T, "
            "Tensor(b!)? cap=None) -> ()")
_LIB.define("swiglu_push(Tensor gu, Tensor? pushes, int T, Tensor(a!)? cap=None) -> Tensor")
_LIB.define("gemm_q8_(Tensor x, Tensor W, Tensor w_scale, Tensor(a!) y, int epilogue, Tensor? pushes, int T, "
            "Tensor(b!)? cap=None) -> ()")
_LIB.define("add_rmsnorm_(Tensor(a!) x, Tensor? y, Tensor w, float eps) -> Tensor")
_LIB.define("add_rmsnorm_split_(Tensor(a!) x, Tensor? y, Tensor w, float eps) -> Tensor")
_LIB.define("argmax_rows_(Tensor x, Tensor(a!) idx) -> ()")
_LIB.define("gemv_norm_(Tensor x, Tensor? x_add, Tensor(b!)? x_out, Tensor norm_w, float eps, Tensor W, "
            "Tensor? w_scale, Tensor(a!) y, int epilogue, Tensor? pushes, int T, Tensor(c!)? cap=None) -> ()")
_LIB.define("gemv_norm_argmax_(Tensor x, Tensor? x_add, Tensor(b!)? x_out, Tensor norm_w, float eps, Tensor W, "
            "Tensor? w_scale, Tensor(a!) y, Tensor(c!) slots, Tensor(d!) idx) -> ()")
_LIB.define("gdn_chunk_prefill_conv_(Tensor y, Tensor conv_w, Tensor? conv_bias, Tensor(a!) conv_state, Tensor A_log, "
            "Tensor dt_bias, int b_off, int a_off, Tensor(b!) state, int Hk, float scale) -> Tensor")
_LIB.define("gdn_decode_sliced_(Tensor y, Tensor A_log, Tensor dt_bias, int b_off, int a_off, Tensor(a!) state, "
            "float scale) -> Tensor")
_LIB.define("gemv_norm_conv_(Tensor x, Tensor? x_add, Tensor(b!)? x_out, Tensor norm_w, float eps, Tensor W, "
            "Tensor? w_scale, Tensor(a!) y, Tensor conv_w, Tensor? conv_bias, Tensor(c!) conv_state) -> ()")
_LIB.define("gemv_gated_norm_(Tensor o, Tensor z, Tensor norm_w, Tensor? head_scale, float eps, Tensor W, "
            "Tensor w_scale, Tensor(a!) y, int epilogue) -> ()")
_LIB.define("attn_prep(Tensor y, Tensor q_norm_w, Tensor k_norm_w, float eps, Tensor cos, Tensor sin, Tensor pos, "
            "Tensor(a!) k_cache, Tensor(b!) v_cache, int Hq, int Hkv, bool want_kv) "
            "-> (Tensor, Tensor, Tensor, Tensor)")


# ---------------------------------------------------------------- gated delta rule
def _gdn_check(q, k, v, g, beta, state):
    _on_gpu(q, k, v, g, beta, state)
    _require(q.dtype in _DT and k.dtype == q.dtype and v.dtype == q.dtype, "q, k, v must share dtype fp32 or bf16")
    _require(g.dtype == torch.float32 and beta.dtype == torch.float32, "g and beta must be fp32")
    _require(q.dim() == 4 and k.shape == q.shape and v.dim() == 4, "q, k: [B, T, Hk, Dk]; v: [B, T, H, Dv]")
    B, T, Hk, Dk = q.shape
    H, Dv = v.shape[2], v.shape[3]
    _require(v.shape[0] == B and v.shape[1] == T, "v must match q in batch and time")
    _require(H % Hk == 0, "value heads must be a multiple of q/k heads")
    _require(tuple(g.shape) == (B, T, H) and tuple(beta.shape) == (B, T, H), "g, beta: [B, T, H]")
    if state is not None:
        _require(state.dtype == torch.float32 and tuple(state.shape) == (B, H, Dk, Dv), "state: [B, H, Dk, Dv] fp32")
    return B, T, Hk, H, Dk, Dv


def _gdn_recurrent_impl(q, k, v, g, beta, initial_state, scale, use_qk_l2norm):
    B, T, Hk, H, Dk, Dv = _gdn_check(q, k, v, g, beta, initial_state)
    o = torch.empty_like(v)
    S = torch.empty(B, H, Dk, Dv, dtype=torch.float32, device=q.device)
    st = _lib.lib().q35_gdn_recurrent(_ptr(q), _ptr(k), _ptr(v), _ptr(g), _ptr(beta), _ptr(initial_state), _ptr(S),
                                      _ptr(o), B, T, Hk, H, Dk, Dv, _DT[q.dtype], float(scale), int(use_qk_l2norm),
                                      _stream(q))
    check(st, "q35_gdn_recurrent")
    return o, S


def _gdn_decode_step_impl(q, k, v, g, beta, state, scale, use_qk_l2norm):
    B, T, Hk, H, Dk, Dv = _gdn_check(q, k, v, g, beta, state)
    o = torch.empty_like(v)
    st = _lib.lib().q35_gdn_recurrent(_ptr(q), _ptr(k), _ptr(v), _ptr(g), _ptr(beta), _ptr(state), _ptr(state),
                                      _ptr(o), B, T, Hk, H, Dk, Dv, _DT[q.dtype], float(scale), int(use_qk_l2norm),
                                      _stream(q))
    check(st, "q35_gdn_recurrent")
    return o


def _gdn_chunk_impl(q, k, v, g, beta, initial_state, chunk_size, scale, use_qk_l2norm):
    B, T, Hk, H, Dk, Dv = _gdn_check(q, k, v, g, beta, initial_state)
    L = _lib.lib()
    nbytes = L.q35_gdn_chunk_workspace_bytes(B, T, H, Dk, Dv, chunk_size, _DT[q.dtype])
    _require(nbytes > 0, f"unsupported chunk prefill shape (Dk={Dk}, Dv={Dv}, chunk={chunk_size})")
    ws = _workspace(nbytes, q.device)
    o = torch.empty_like(v)
    S = torch.empty(B, H, Dk, Dv, dtype=torch.float32, device=q.device)
    st = L.q35_gdn_chunk_prefill(_ptr(q), _ptr(k), _ptr(v), _ptr(g), _ptr(beta), _ptr(initial_state), _ptr(S),
                                 _ptr(o), B, T, Hk, H, Dk, Dv, _DT[q.dtype], float(scale), int(use_qk_l2norm),
                                 chunk_size, _ptr(ws), ws.numel(), _stream(q))
    check(st, "q35_gdn_chunk_prefill")
    return o, S


# ---------------------------------------------------------------- gated attention
def _tables_check(cos, sin, rows_needed):
    _require(cos.dtype == torch.float32 and sin.dtype == torch.float32, "cos/sin tables must be fp32")
    _require(cos.dim() == 2 and sin.shape == cos.shape, "cos/sin tables: [P, rot/2]")
    _require(cos.shape[0] >= rows_needed or cos.shape[1] == 0, f"cos/sin tables need {rows_needed} rows")
    return 2 * cos.shape[1]


def _attn_prefill_impl(q, k, v, gate, cos, sin, pos0, scale):
    _on_gpu(q, k, v, gate, cos, sin)
    _require(q.dtype == torch.bfloat16 and k.dtype == q.dtype and v.dtype == q.dtype and gate.dtype == q.dtype,
             "q, k, v, gate must be bf16")
    _require(q.dim() == 4 and k.dim() == 4 and v.shape == k.shape, "q: [B, T, Hq, D]; k, v: [B, T, Hkv, D]")
    B, T, Hq, D = q.shape
    Hkv = k.shape[2]
    _require(k.shape[0] == B and k.shape[1] == T and k.shape[3] == D, "k/v must match q in batch, time, head dim")
    _require(tuple(gate.shape) == (B, T, Hq * D), "gate: [B, T, Hq * D]")
    rot = _tables_check(cos, sin, pos0 + T)
    out = torch.empty(B, T, Hq * D, dtype=q.dtype, device=q.device)
    L = _lib.lib()
    nbytes = L.q35_gated_attn_prefill_workspace_bytes(B, T, Hq, Hkv, D)
    _require(nbytes > 0, "unsupported attention shape")
    ws = _workspace(nbytes, q.device)
    st = L.q35_gated_attn_prefill(_ptr(q), _ptr(k), _ptr(v), _ptr(gate), _ptr(cos), _ptr(sin), int(pos0),
                                  _ptr(out), B, T, Hq, Hkv, D, rot, float(scale), _ptr(ws), ws.numel(), _stream(q))
    check(st, "q35_gated_attn_prefill")
    return out


def _attn_prefill_cached_impl(q, k_cache, v_cache, gate, pos, cos, sin, scale):
    _on_gpu(q, k_cache, v_cache, gate, pos, cos, sin)
    _require(q.dtype == torch.bfloat16 and k_cache.dtype == q.dtype and v_cache.dtype == q.dtype
             and gate.dtype == q.dtype, "q, caches, gate must be bf16")
    _require(q.dim() == 4 and k_cache.dim() == 4 and v_cache.shape == k_cache.shape,
             "q: [B, T, Hq, D]; caches: [B, Hkv, max_len, D]")
    B, T, Hq, D = q.shape
    Hkv, max_len = k_cache.shape[1], k_cache.shape[2]
    _require(k_cache.shape[0] == B and k_cache.shape[3] == D, "caches must match q in batch and head dim")
    _require(tuple(gate.shape) == (B, T, Hq * D), "gate: [B, T, Hq * D]")
    _require(pos.dtype == torch.int32 and tuple(pos.shape) == (B,), "pos: [B] int32")
    _require(max_len % 64 == 0, "the cache length must be a multiple of 64 for a multi-token call over the cache")
    _require(T <= max_len, "more tokens than the cache holds")
    rot = _tables_check(cos, sin, max_len)
    L = _lib.lib()
    nbytes = L.q35_gated_attn_prefill_cached_workspace_bytes(B, Hkv, D, max_len)
    _require(nbytes > 0, "unsupported attention shape")
    ws = _workspace(nbytes, q.device)
    out = torch.empty(B, T, Hq * D, dtype=q.dtype, device=q.device)
    st = L.q35_gated_attn_prefill_cached(_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(gate), _ptr(pos), _ptr(cos),
                                         _ptr(sin), _ptr(out), B, T, Hq, Hkv, D, max_len, rot, float(scale),
                                         _ptr(ws), ws.numel(), _stream(q))
    check(st, "q35_gated_attn_prefill_cached")
    return out


def _attn_decode_impl(q, k_cache, v_cache, gate, cache_len, cos, sin, scale, splits, f32_out=False):
    _on_gpu(q, k_cache, v_cache, gate, cache_len, cos, sin)
    _require(q.dtype == torch.bfloat16 and k_cache.dtype == q.dtype and v_cache.dtype == q.dtype
             and gate.dtype == q.dtype, "q, caches, gate must be bf16")
    _require(cache_len.dtype == torch.int32, "cache_len must be int32")
    _require(q.dim() == 3 and k_cache.dim() == 4 and v_cache.shape == k_cache.shape,
             "q: [B, Hq, D]; caches: [B, Hkv, max_len, D]")
    B, Hq, D = q.shape
    Hkv, max_len = k_cache.shape[1], k_cache.shape[2]
    _require(k_cache.shape[0] == B and k_cache.shape[3] == D, "caches must match q in batch and head dim")
    _require(tuple(gate.shape) == (B, Hq * D) and tuple(cache_len.shape) == (B,), "gate: [B, Hq*D]; cache_len: [B]")
    rot = _tables_check(cos, sin, max_len)
    L = _lib.lib()
    nbytes = L.q35_gated_attn_decode_workspace_bytes(B, Hq, Hkv, D, max_len, splits)
    ws = _workspace(nbytes, q.device)
    odt = torch.float32 if f32_out else q.dtype
    out = torch.empty(B, Hq * D, dtype=odt, device=q.device)
    st = L.q35_gated_attn_decode(_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(gate), _ptr(cache_len), _ptr(cos),
                                 _ptr(sin), _ptr(out), _DT[odt], B, Hq, Hkv, D, max_len, rot, float(scale), int(splits),
                                 _ptr(ws), ws.numel(), _stream(q))
    check(st, "q35_gated_attn_decode")
    return out


def _attn_decode_proj_impl(y, q_norm_w, k_norm_w, eps, k_cache, v_cache, pos, cos, sin, Hq, scale, splits,
                           f32_out=False):
    _on_gpu(q_norm_w, k_norm_w, k_cache, v_cache, pos, cos, sin)
    _require(y.is_cuda and y.dtype == torch.float32 and y.is_contiguous() and y.dim() in (2, 3)
             and (y.dim() == 2 or y.shape[1] == 1), "y: [B, W] or [B, 1, W] fp32 dense (the fused projection output)")
    y2 = y.view(y.shape[0], y.shape[-1])
    B, W = y2.shape
    _require(k_cache.dtype == torch.bfloat16 and k_cache.dim() == 4 and v_cache.shape == k_cache.shape
             and v_cache.dtype == k_cache.dtype, "caches: [B, Hkv, max_len, D] bf16")
    Hkv, max_len, D = k_cache.shape[1], k_cache.shape[2], k_cache.shape[3]
    _require(k_cache.shape[0] == B, "caches must match y in batch")
    _require(pos.dtype == torch.int32 and tuple(pos.shape) == (B,), "pos: [B] int32")
    _require(q_norm_w.dtype == torch.float32 and k_norm_w.dtype == torch.float32 and q_norm_w.numel() == D
             and k_norm_w.numel() == D and q_norm_w.is_contiguous() and k_norm_w.is_contiguous(),
             "q_norm_w, k_norm_w: [D] fp32")
    rot = _tables_check(cos, sin, max_len)
    L = _lib.lib()
    ws = _workspace(L.q35_gated_attn_decode_workspace_bytes(B, Hq, Hkv, D, max_len, splits), y.device)
    odt = torch.float32 if f32_out else torch.bfloat16
    out = torch.empty(B, Hq * D, dtype=odt, device=y.device)
    st = L.q35_gated_attn_decode_proj(_ptr(y2), W, _ptr(q_norm_w), _ptr(k_norm_w), float(eps), _ptr(k_cache),
                                      _ptr(v_cache), _ptr(pos), _ptr(cos), _ptr(sin), _ptr(out), _DT[odt], B, Hq, Hkv,
                                      D, max_len, rot, float(scale), int(splits), _ptr(ws), ws.numel(), _stream(y))
    check(st, "q35_gated_attn_decode_proj")
    return out


def _attn_prefill_proj_impl(y, q_norm_w, k_norm_w, eps, k_cache, v_cache, pos0, cos, sin, Hq, scale):
    _on_gpu(q_norm_w, k_norm_w, k_cache, v_cache, cos, sin)
    _require(y.is_cuda and y.dtype == torch.float32 and y.dim() == 3 and y.stride(2) == 1
             and y.stride(0) == y.shape[1] * y.stride(1), "y: [B, T, W] fp32 with dense rows (the fused projection "
             "output)")
    B, T, W = y.shape
    ldy = y.stride(1)
    _require(k_cache.dtype == torch.bfloat16 and k_cache.dim() == 4 and v_cache.shape == k_cache.shape
             and v_cache.dtype == k_cache.dtype and k_cache.is_contiguous() and v_cache.is_contiguous(),
             "caches: [B, Hkv, max_len, D] bf16 dense")
    Hkv, max_len, D = k_cache.shape[1], k_cache.shape[2], k_cache.shape[3]
    _require(k_cache.shape[0] == B, "caches must match y in batch")
    _require(W >= Hq * 2 * D + 2 * Hkv * D, "y: too narrow for [q | gate] x Hq, k, v")
    _require(q_norm_w.dtype == torch.float32 and k_norm_w.dtype == torch.float32 and q_norm_w.numel() == D
             and k_norm_w.numel() == D and q_norm_w.is_contiguous() and k_norm_w.is_contiguous(),
             "q_norm_w, k_norm_w: [D] fp32")
    _require(0 <= pos0 and pos0 + T <= max_len, f"positions {pos0}..{pos0 + T - 1} exceed the cache ({max_len})")
    rot = _tables_check(cos, sin, pos0 + T)
    L = _lib.lib()
    nbytes = L.q35_gated_attn_prefill_proj_workspace_bytes(B, T, Hq, Hkv, D)
    _require(nbytes > 0, "unsupported attention shape")
    ws = _workspace(nbytes, y.device)
    out = torch.empty(B, T, Hq * D, dtype=torch.bfloat16, device=y.device)
    st = L.q35_gated_attn_prefill_proj(_ptr(y), ldy, _ptr(q_norm_w), _ptr(k_norm_w), float(eps), _ptr(k_cache),
                                       _ptr(v_cache), int(pos0), _ptr(cos), _ptr(sin), _ptr(out), B, T, Hq, Hkv, D,
                                       max_len, rot, float(scale), _ptr(ws), ws.numel(), _stream(y))
    check(st, "q35_gated_attn_prefill_proj")
    return out


def _attn_prefill_cached_proj_impl(y, q_norm_w, k_norm_w, eps, k_cache, v_cache, pos, cos, sin, Hq, scale):
    _on_gpu(q_norm_w, k_norm_w, k_cache, v_cache, pos, cos, sin)
    _require(y.is_cuda and y.dtype == torch.float32 and y.dim() == 3 and y.stride(2) == 1
             and y.stride(0) == y.shape[1] * y.stride(1), "y: [B, T, W] fp32 with dense rows (the fused projection "
             "output)")
    B, T, W = y.shape
    ldy = y.stride(1)
    _require(k_cache.dtype == torch.bfloat16 and k_cache.dim() == 4 and v_cache.shape == k_cache.shape
             and v_cache.dtype == k_cache.dtype and k_cache.is_contiguous() and v_cache.is_contiguous(),
             "caches: [B, Hkv, max_len, D] bf16 dense")
    Hkv, max_len, D = k_cache.shape[1], k_cache.shape[2], k_cache.shape[3]
    _require(k_cache.shape[0] == B, "caches must match y in batch")
    _require(W >= Hq * 2 * D + 2 * Hkv * D, "y: too narrow for [q | gate] x Hq, k, v")
    _require(q_norm_w.dtype == torch.float32 and k_norm_w.dtype == torch.float32 and q_norm_w.numel() == D
             and k_norm_w.numel() == D and q_norm_w.is_contiguous() and k_norm_w.is_contiguous(),
             "q_norm_w, k_norm_w: [D] fp32")
    _require(pos.dtype == torch.int32 and tuple(pos.shape) == (B,), "pos: [B] int32")
    _require(max_len % 64 == 0, "the cache length must be a multiple of 64 for a multi-token call over the cache")
    _require(T <= max_len, "more tokens than the cache holds")
    rot = _tables_check(cos, sin, max_len)
    L = _lib.lib()
    nbytes = L.q35_gated_attn_prefill_cached_proj_workspace_bytes(B, T, Hq, Hkv, D, max_len)
    _require(nbytes > 0, "unsupported attention shape")
    ws = _workspace(nbytes, y.device)
    out = torch.empty(B, T, Hq * D, dtype=torch.bfloat16, device=y.device)
    st = L.q35_gated_attn_prefill_cached_proj(_ptr(y), ldy, _ptr(q_norm_w), _ptr(k_norm_w), float(eps),
                                              _ptr(k_cache), _ptr(v_cache), _ptr(pos), _ptr(cos), _ptr(sin), _ptr(out),
                                              B, T, Hq, Hkv, D, max_len, rot, float(scale), _ptr(ws), ws.numel(),
                                              _stream(y))
    check(st, "q35_gated_attn_prefill_cached_proj")
    return out


def _resid_add_impl(x, vecs, vec_of_row):
    _on_gpu(x, vecs, vec_of_row)
    _require(x.dtype in _DT and vecs.dtype == torch.float32, "x fp32/bf16, vecs fp32")
    _require(x.dim() == 3 and vecs.dim() == 2 and vecs.shape[1] == x.shape[2], "x: [rows, T, H]; vecs: [nvec, H]")
    if vec_of_row is not None:
        _require(vec_of_row.dtype == torch.int32 and tuple(vec_of_row.shape) == (x.shape[0],),
                 "vec_of_row: [rows] int32")
    rows, T, H = x.shape
    st = _lib.lib().q35_resid_add_rows(_ptr(x), _ptr(vecs), _ptr(vec_of_row), rows, T, H, vecs.shape[0],
                                       _DT[x.dtype], _stream(x))
    check(st, "q35_resid_add_rows")


# ---------------------------------------------------------------- layer front ends
def _rows_view(t, width, what):
    """A [..., width] fp32 view whose rows are evenly strided and whose last dim is dense: (rows, row stride)."""
    _require(t.is_cuda and t.dtype == torch.float32, f"{what} must be an fp32 HIP tensor")
    _require(t.shape[-1] == width and t.stride(-1) == 1, f"{what}: last dim {width}, dense")
    rows = t.numel() // max(width, 1)
    if t.dim() == 1:
        return rows, width
    flat = t.reshape(-1, width) if t.dim() > 2 else t
    _require(flat.data_ptr() == t.data_ptr() and (rows <= 1 or flat.stride(0) >= width),
             f"{what}: rows must be evenly strided")
    return rows, flat.stride(0)


def _gdn_conv_impl(y, conv_w, conv_bias, conv_state, A_log, dt_bias, b_off, a_off, Hk, dk, Hv, dv, bf16_out):
    _on_gpu(conv_w, conv_bias, conv_state, A_log, dt_bias)
    _require(y.is_cuda and y.dtype == torch.float32 and y.dim() == 3 and y.is_contiguous(),
             "y: [B, T, W] fp32 dense (the fused projection output)")
    B, T, W = y.shape
    C = 2 * Hk * dk + Hv * dv
    _require(conv_w.dim() == 2 and conv_w.shape[0] == C and conv_w.dtype == torch.float32, "conv_w: [C, K] fp32")
    K = conv_w.shape[1]
    _require(conv_state.dtype == torch.float32 and tuple(conv_state.shape) == (B, K - 1, C),
             "conv_state: [B, K - 1, C] fp32")
    _require(A_log.numel() == Hv and dt_bias.numel() == Hv, "A_log, dt_bias: [Hv]")
    dt = torch.bfloat16 if bf16_out else torch.float32
    q = torch.empty(B, T, Hk, dk, dtype=dt, device=y.device)
    k = torch.empty_like(q)
    v = torch.empty(B, T, Hv, dv, dtype=dt, device=y.device)
    g = torch.empty(B, T, Hv, dtype=torch.float32, device=y.device)
    beta = torch.empty_like(g)
    st = _lib.lib().q35_gdn_conv(_ptr(y), W, _ptr(conv_w), _ptr(conv_bias), _ptr(conv_state), _ptr(A_log),
                                 _ptr(dt_bias), int(b_off), int(a_off), _ptr(q), _ptr(k), _ptr(v), _ptr(g),
                                 _ptr(beta), B, T, Hk, dk, Hv, dv, K, _DT[dt], _stream(y))
    check(st, "q35_gdn_conv")
    return q, k, v, g, beta


def _gdn_decode_fused_impl(y, conv_w, conv_bias, conv_state, A_log, dt_bias, b_off, a_off, z_off, state, norm_w,
                           head_scale, eps, scale):
    _on_gpu(conv_w, conv_bias, conv_state, A_log, dt_bias, state, norm_w, head_scale)
    _require(y.is_cuda and y.dtype == torch.float32 and y.dim() == 2 and y.stride(1) == 1,
             "y: [B, W] fp32 with unit column stride (one projection row per sequence)")
    B, W = y.shape
    _require(state.dtype == torch.float32 and state.dim() == 4 and state.is_contiguous()
             and state.shape[0] == B and state.shape[2] == state.shape[3], "state: [B, H, d, d] fp32 dense")
    H, d = state.shape[1], state.shape[2]
    C = 3 * H * d
    _require(conv_w.dim() == 2 and conv_w.shape[0] == C and conv_w.dtype == torch.float32 and conv_w.is_contiguous(),
             "conv_w: [C, K] fp32 dense")
    K = conv_w.shape[1]
    _require(conv_state.dtype == torch.float32 and tuple(conv_state.shape) == (B, K - 1, C)
             and conv_state.is_contiguous(), "conv_state: [B, K - 1, C] fp32 dense")
    _require(A_log.numel() == H and dt_bias.numel() == H and norm_w.numel() == d, "A_log, dt_bias: [H]; norm_w: [d]")
    for t in (A_log, dt_bias, norm_w, head_scale):
        _require(t is None or (t.dtype == torch.float32 and t.is_contiguous()), "gate and norm tensors: fp32 dense")
    if head_scale is not None:
        _require(head_scale.numel() == H, "head_scale: [H]")
    out = torch.empty(B, H * d, dtype=torch.float32, device=y.device)
    st = _lib.lib().q35_gdn_decode_fused(_ptr(y), y.stride(0), _ptr(conv_w), _ptr(conv_bias), _ptr(conv_state),
                                         _ptr(A_log), _ptr(dt_bias), int(b_off), int(a_off), int(z_off), _ptr(state),
                                         _ptr(norm_w), _ptr(head_scale), float(eps), float(scale), _ptr(out), B, H, d,
                                         K, _stream(y))
    check(st, "q35_gdn_decode_fused")
    return out


def _gdn_chunk_prefill_conv_impl(y, conv_w, conv_bias, conv_state, A_log, dt_bias, b_off, a_off, state, Hk, scale):
    _on_gpu(conv_w, conv_bias, conv_state, A_log, dt_bias, state)
    _require(y.is_cuda and y.dtype == torch.float32 and y.dim() == 3 and y.is_contiguous(),
             "y: [B, T, W] fp32 dense (the fused projection output)")
    B, T, W = y.shape
    _require(state.dtype == torch.float32 and state.dim() == 4 and state.is_contiguous() and state.shape[0] == B
             and state.shape[2] == state.shape[3], "state: [B, H, d, d] fp32 dense")
    H, d = state.shape[1], state.shape[2]
    C = (2 * Hk + H) * d
    _require(conv_w.dim() == 2 and conv_w.shape[0] == C and conv_w.dtype == torch.float32, "conv_w: [C, K] fp32")
    K = conv_w.shape[1]
    _require(conv_state.dtype == torch.float32 and tuple(conv_state.shape) == (B, K - 1, C),
             "conv_state: [B, K - 1, C] fp32")
    _require(A_log.numel() == H and dt_bias.numel() == H, "A_log, dt_bias: [H]")
    L = _lib.lib()
    nbytes = L.q35_gdn_chunk_workspace_bytes(B, T, H, d, d, 64, _DT[torch.float32])
    _require(nbytes > 0, f"unsupported chunk prefill shape (d={d})")
    ws = _workspace(nbytes, y.device)
    o = torch.empty(B, T, H, d, dtype=torch.float32, device=y.device)
    st = L.q35_gdn_chunk_prefill_conv(_ptr(y), W, _ptr(conv_w), _ptr(conv_bias), _ptr(conv_state), _ptr(A_log),
                                      _ptr(dt_bias), int(b_off), int(a_off), _ptr(state), _ptr(state), _ptr(o), B, T,
                                      int(Hk), H, d, d, K, float(scale), _ptr(ws), ws.numel(), _stream(y))
    check(st, "q35_gdn_chunk_prefill_conv")
    return o


def _gdn_decode_sliced_impl(y, A_log, dt_bias, b_off, a_off, state, scale):
    _on_gpu(A_log, dt_bias, state)
    _require(y.is_cuda and y.dtype == torch.float32 and y.dim() == 2 and y.stride(1) == 1,
             "y: [B, W] fp32 with unit column stride (one projection row per sequence)")
    B = y.shape[0]
    _require(state.dtype == torch.float32 and state.dim() == 4 and state.is_contiguous()
             and state.shape[0] == B and state.shape[2] == state.shape[3], "state: [B, H, d, d] fp32 dense")
    H, d = state.shape[1], state.shape[2]
    _require(A_log.numel() == H and dt_bias.numel() == H and A_log.dtype == torch.float32
             and dt_bias.dtype == torch.float32 and A_log.is_contiguous() and dt_bias.is_contiguous(),
             "A_log, dt_bias: [H] fp32 dense")
    out = torch.empty(B, H * d, dtype=torch.float32, device=y.device)
    st = _lib.lib().q35_gdn_decode_sliced(_ptr(y), y.stride(0), _ptr(A_log), _ptr(dt_bias), int(b_off), int(a_off),
                                          _ptr(state), float(scale), _ptr(out), B, H, d, _stream(y))
    check(st, "q35_gdn_decode_sliced")
    return out


def _gated_rmsnorm_impl(o, z, w, head_scale, eps, split=False):
    _on_gpu(o, w, head_scale)
    _require(o.dtype in _DT and o.dim() >= 2, "o: [..., Hv, dv] fp32 or bf16")
    _require(not split or o.dtype == torch.float32, "the split output form takes fp32 o")
    Hv, dv = o.shape[-2], o.shape[-1]
    M = o.numel() // (Hv * dv)
    rows, ldz = _rows_view(z, Hv * dv, "z")
    _require(rows == M, "z must have one row per token of o")
    _require(w.numel() == dv and w.dtype == torch.float32, "w: [dv] fp32")
    if head_scale is not None:
        _require(head_scale.numel() == Hv and head_scale.dtype == torch.float32, "head_scale: [Hv] fp32")
    out = torch.empty(*o.shape[:-2], Hv * dv, dtype=torch.int32 if split else o.dtype, device=o.device)
    if split:
        st = _lib.lib().q35_gated_rmsnorm_split(_ptr(o), _ptr(z), ldz, _ptr(w), _ptr(head_scale), _ptr(out), M, Hv,
                                                dv, float(eps), _stream(o))
        check(st, "q35_gated_rmsnorm_split")
        return out
    st = _lib.lib().q35_gated_rmsnorm(_ptr(o), _ptr(z), ldz, _ptr(w), _ptr(head_scale), _ptr(out), M, Hv, dv,
                                      float(eps), _DT[o.dtype], _stream(o))
    check(st, "q35_gated_rmsnorm")
    return out


def _gated_rmsnorm_split_impl(o, z, w, head_scale, eps):
    return _gated_rmsnorm_impl(o, z, w, head_scale, eps, split=True)


def _attn_prep_impl(y, q_norm_w, k_norm_w, eps, cos, sin, pos, k_cache, v_cache, Hq, Hkv, want_kv):
    _on_gpu(q_norm_w, k_norm_w, cos, sin, pos, k_cache, v_cache)
    _require(y.is_cuda and y.dtype == torch.float32 and y.dim() == 3 and y.is_contiguous(),
             "y: [B, T, W] fp32 dense (the fused projection output)")
    B, T, W = y.shape
    _require(k_cache.dtype == torch.bfloat16 and v_cache.shape == k_cache.shape and k_cache.dim() == 4,
             "caches: [B, Hkv, max_len, D] bf16")
    _require(k_cache.shape[0] == B and k_cache.shape[1] == Hkv, "caches must match the batch and kv heads")
    D, max_len = k_cache.shape[3], k_cache.shape[2]
    _require(pos.dtype == torch.int32 and tuple(pos.shape) == (B,), "pos: [B] int32")
    rot = _tables_check(cos, sin, max_len)
    q = torch.empty(B, T, Hq, D, dtype=torch.bfloat16, device=y.device)
    gate = torch.empty(B, T, Hq * D, dtype=torch.bfloat16, device=y.device)
    if want_kv:
        k = torch.empty(B, T, Hkv, D, dtype=torch.bfloat16, device=y.device)
        v = torch.empty_like(k)
    else:
        k = v = torch.empty(0, dtype=torch.bfloat16, device=y.device)
    st = _lib.lib().q35_attn_prep(_ptr(y), W, _ptr(q_norm_w), _ptr(k_norm_w), float(eps), _ptr(cos), _ptr(sin), rot,
                                  _ptr(pos), _ptr(q), _ptr(gate), _ptr(k) if want_kv else None,
                                  _ptr(v) if want_kv else None, _ptr(k_cache), _ptr(v_cache), max_len, B, T, Hq, Hkv,
                                  D, _stream(y))
    check(st, "q35_attn_prep")
    return q, gate, k, v


# ---------------------------------------------------------------- decode matrix-vector products, SwiGLU hook
# limits of the conv epilogue of the decode GEMV (q35_gemv_norm_conv): conv taps, and output rows (1024 tiles of 16
# rows, or of 8 rows for more than 4 rows of x)
GEMV_CONV_MAX_K = 8


def gemv_conv_max_n(M):
    return 1024 * (8 if M > 4 else 16)
# "add_fixed": accumulate with every output summed in one fixed order (repeatable bits; no split over K)
_EPI = {"store": 0, "add": 1, "swiglu": 2, "add_fixed": 4}


def _pushes_check(pushes):
    if pushes is None:
        return 0
    _require(pushes.dtype == torch.int32 and pushes.dim() == 2 and pushes.shape[1] == 6 and pushes.is_contiguous(),
             "pushes: [n, 6] int32 records (see pack_pushes)")
    return pushes.shape[0]


def _cap_args(cap, M, T, I, device):
    """(pointer, ld_cap, ld_cap_row) of a capture destination: a view [R, T, I] (R * T = M rows; any row and token
    strides, unit neuron stride) or [M, I] (unit neuron stride) fp32 on the product's device; None -> no capture."""
    if cap is None:
        return None, 0, 0
    _require(cap.is_cuda and cap.device == device and cap.dtype == torch.float32 and cap.stride(-1) == 1,
             "capture: fp32 view on the product's device with unit neuron stride")
    if cap.dim() == 3:
        _require(cap.shape[0] * cap.shape[1] == M and cap.shape[1] == T and cap.shape[2] == I,
                 "capture: [rows, T, I] with rows * T = M")
        return cap.data_ptr(), cap.stride(1), cap.stride(0)
    _require(cap.dim() == 2 and cap.shape[0] == M and cap.shape[1] == I, "capture: [M, I] or [rows, T, I]")
    return cap.data_ptr(), cap.stride(0), cap.stride(0) * T


def _weight_format(W, w_scale, N, K):
    """The C ABI's weight format code of (W, w_scale): fp32 W (no scale) -> Q35_F32; int8 W with w_scale [N] fp32 ->
    Q35_I8 (one scale per output row); int8 W with w_scale [N, K / 128] fp32 -> Q35_I8_G128 (one scale per group of
    128 inputs, the engine's q8 format)."""
    if W.dtype == torch.float32:
        _require(w_scale is None, "fp32 W takes no w_scale")
        return Q35_F32
    _require(w_scale is not None and w_scale.dtype == torch.float32 and w_scale.is_contiguous(),
             "int8 W needs a contiguous fp32 w_scale")
    if w_scale.dim() == 2:
        _require(K % 128 == 0 and tuple(w_scale.shape) == (N, K // 128),
                 "group scales: w_scale [N, K / 128] fp32 (K a multiple of 128)")
        return Q35_I8_G128
    _require(w_scale.dim() == 1 and w_scale.numel() == N, "per-row scales: w_scale [N] fp32")
    return Q35_I8


def _gemv_impl(x, W, w_scale, y, epilogue, pushes, T, cap=None):
    _on_gpu(x, W, w_scale, y, pushes)
    _require(x.dtype == torch.float32 and x.dim() == 2 and y.dtype == torch.float32 and y.dim() == 2,
             "x: [M, K] fp32; y: [M, N or N/2] fp32")
    _require(W.dim() == 2 and W.dtype in (torch.int8, torch.float32), "W: [N, K] int8 or fp32")
    M, K = x.shape
    N = W.shape[0]
    _require(W.shape[1] == K and y.shape[0] == M, "x, W, y shapes disagree")
    _require(y.shape[1] == (N // 2 if epilogue == 2 else N), "y: [M, N] ([M, N / 2] for the SwiGLU epilogue)")
    fmt = _weight_format(W, w_scale, N, K)
    npush = _pushes_check(pushes)
    _require(cap is None or epilogue == 2, "capture: SwiGLU epilogue only")
    cp, ldc, ldcr = _cap_args(cap, M, int(T), N // 2, x.device)
    st = _lib.lib().q35_gemv(_ptr(x), K, _ptr(W), fmt, _ptr(w_scale), _ptr(y), y.shape[1], M, N, K, int(epilogue),
                             _ptr(pushes), npush, int(T), cp, ldc, ldcr, _stream(x))
    check(st, "q35_gemv")


def _gemm_q8_impl(x, W, w_scale, y, epilogue, pushes, T, cap=None):
    _on_gpu(W, w_scale, pushes)
    _require(x.is_cuda and x.dtype in (torch.float32, torch.int32, torch.bfloat16) and x.dim() == 2
             and x.stride(1) == 1, "x: [M, K] fp32, bf16 or int32 words of split activations, unit column stride")
    _require(y.is_cuda and y.dtype == (torch.int32 if epilogue == 3 else torch.float32) and y.dim() == 2
             and y.stride(1) == 1, "y: [M, N] fp32 (int32 words of split activations for epilogue 3)")
    _require(W.dim() == 2 and W.dtype == torch.int8, "W: [N, K] int8")
    M, K = x.shape
    N = W.shape[0]
    _require(W.shape[1] == K and y.shape[0] == M, "x, W, y shapes disagree")
    _require(y.shape[1] == (N // 2 if epilogue in (2, 3) else N), "y: [M, N] ([M, N / 2] for the SwiGLU epilogue)")
    fmt = _weight_format(W, w_scale, N, K)
    _require(K % 64 == 0, "K must be a multiple of 64")
    npush = _pushes_check(pushes)
    fn = {torch.int32: "q35_gemm_q8_split", torch.bfloat16: "q35_gemm_q8_bf16"}.get(x.dtype, "q35_gemm_q8")
    _require(cap is None or epilogue in (2, 3), "capture: SwiGLU epilogues only")
    cp, ldc, ldcr = _cap_args(cap, M, int(T), N // 2, x.device)
    st = getattr(_lib.lib(), fn)(_ptr(x), x.stride(0), _ptr(W), fmt, _ptr(w_scale), _ptr(y), y.stride(0), M, N, K,
                                 int(epilogue), _ptr(pushes), npush, int(T), cp, ldc, ldcr, _stream(x))
    check(st, fn)


def _gemv_norm_impl(x, x_add, x_out, norm_w, eps, W, w_scale, y, epilogue, pushes, T, cap=None):
    _on_gpu(x, x_add, x_out, norm_w, W, w_scale, y, pushes)
    _require(x.dtype == torch.float32 and x.dim() == 2 and y.dtype == torch.float32 and y.dim() == 2,
             "x: [M, K] fp32; y: [M, N or N/2] fp32")
    M, K = x.shape
    for t in (x_add, x_out):
        _require(t is None or (t.dtype == torch.float32 and tuple(t.shape) == (M, K) and t.stride(0) == x.stride(0)
                               and t.stride(1) == 1), "x_add / x_out: like x")
    _require(norm_w.dtype == torch.float32 and norm_w.numel() == K and norm_w.is_contiguous(), "norm_w: [K] fp32")
    _require(W.dim() == 2 and W.dtype in (torch.int8, torch.float32) and W.shape[1] == K, "W: [N, K] int8 or fp32")
    N = W.shape[0]
    _require(y.shape[0] == M and y.shape[1] == (N // 2 if epilogue == 2 else N), "y: [M, N] ([M, N / 2] SwiGLU)")
    fmt = _weight_format(W, w_scale, N, K)
    _require(cap is None or epilogue == 2, "capture: SwiGLU epilogue only")
    cp, ldc, ldcr = _cap_args(cap, M, int(T), N // 2, x.device)
    st = _lib.lib().q35_gemv_norm(_ptr(x), _ptr(x_add), _ptr(x_out), x.stride(0), _ptr(norm_w), float(eps), _ptr(W),
                                  fmt, _ptr(w_scale), _ptr(y), y.shape[1], M, N, K, int(epilogue), _ptr(pushes),
                                  _pushes_check(pushes), int(T), cp, ldc, ldcr, _stream(x))
    check(st, "q35_gemv_norm")


def _gemv_norm_argmax_impl(x, x_add, x_out, norm_w, eps, W, w_scale, y, slots, idx):
    _on_gpu(x, x_add, x_out, norm_w, W, w_scale, y, slots, idx)
    _require(x.dtype == torch.float32 and x.dim() == 2 and y.dtype == torch.float32 and y.dim() == 2,
             "x: [M, K] fp32; y: [M, N] fp32")
    M, K = x.shape
    for t in (x_add, x_out):
        _require(t is None or (t.dtype == torch.float32 and tuple(t.shape) == (M, K) and t.stride(0) == x.stride(0)
                               and t.stride(1) == 1), "x_add / x_out: like x")
    _require(norm_w.dtype == torch.float32 and norm_w.numel() == K and norm_w.is_contiguous(), "norm_w: [K] fp32")
    _require(W.dim() == 2 and W.dtype in (torch.int8, torch.float32) and W.shape[1] == K, "W: [N, K] int8 or fp32")
    N = W.shape[0]
    _require(tuple(y.shape) == (M, N) and y.stride(1) == 1, "y: [M, N] fp32")
    _require(slots.dtype == torch.int64 and slots.numel() == M and slots.is_contiguous(),
             "slots: [M] int64, zeros before the first call (each call leaves them zero)")
    _require(idx.dtype == torch.int32 and idx.numel() == M and idx.is_contiguous(), "idx: [M] int32")
    fmt = _weight_format(W, w_scale, N, K)
    st = _lib.lib().q35_gemv_norm_argmax(_ptr(x), _ptr(x_add), _ptr(x_out), x.stride(0), _ptr(norm_w), float(eps),
                                         _ptr(W), fmt, _ptr(w_scale), _ptr(y), y.stride(0), M, N, K, _ptr(slots),
                                         _ptr(idx), _stream(x))
    check(st, "q35_gemv_norm_argmax")


def _gemv_norm_conv_impl(x, x_add, x_out, norm_w, eps, W, w_scale, y, conv_w, conv_bias, conv_state):
    _on_gpu(x, x_add, x_out, norm_w, W, w_scale, y, conv_w, conv_bias, conv_state)
    _require(x.dtype == torch.float32 and x.dim() == 2 and y.dtype == torch.float32 and y.dim() == 2,
             "x: [M, K] fp32; y: [M, N] fp32")
    M, K = x.shape
    for t in (x_add, x_out):
        _require(t is None or (t.dtype == torch.float32 and tuple(t.shape) == (M, K) and t.stride(0) == x.stride(0)
                               and t.stride(1) == 1), "x_add / x_out: like x")
    _require(norm_w.dtype == torch.float32 and norm_w.numel() == K and norm_w.is_contiguous(), "norm_w: [K] fp32")
    _require(W.dim() == 2 and W.dtype in (torch.int8, torch.float32) and W.shape[1] == K, "W: [N, K] int8 or fp32")
    N = W.shape[0]
    _require(y.shape[0] == M and y.shape[1] == N and y.stride(1) == 1, "y: [M, N] with unit column stride")
    _require(conv_w.dtype == torch.float32 and conv_w.dim() == 2 and conv_w.is_contiguous(), "conv_w: [C, K] fp32")
    C, Kc = conv_w.shape
    _require(conv_bias is None or (conv_bias.dtype == torch.float32 and conv_bias.numel() == C), "conv_bias: [C]")
    _require(conv_state.dtype == torch.float32 and tuple(conv_state.shape) == (M, Kc - 1, C)
             and conv_state.is_contiguous(), "conv_state: [M, K - 1, C] fp32 dense")
    fmt = _weight_format(W, w_scale, N, K)
    st = _lib.lib().q35_gemv_norm_conv(_ptr(x), _ptr(x_add), _ptr(x_out), x.stride(0), _ptr(norm_w), float(eps),
                                       _ptr(W), fmt, _ptr(w_scale), _ptr(y), y.stride(0), M, N, K, _ptr(conv_w),
                                       _ptr(conv_bias), _ptr(conv_state), C, Kc, _stream(x))
    check(st, "q35_gemv_norm_conv")


def _gemv_gated_norm_impl(o, z, norm_w, head_scale, eps, W, w_scale, y, epilogue):
    _on_gpu(o, norm_w, head_scale, W, w_scale, y)
    _require(z.is_cuda and z.device == o.device, "z must be on o's device (rows may be strided)")
    _require(o.dtype == torch.float32 and o.dim() == 2 and o.stride(1) == 1 and z.dtype == torch.float32
             and z.dim() == 2 and z.stride(1) == 1 and z.shape[0] == o.shape[0] and z.shape[1] >= o.shape[1],
             "o: [M, K] fp32; z: [M, >= K] fp32, unit column strides")
    M, K = o.shape
    _require(norm_w.dtype == torch.float32 and norm_w.numel() == 128 and norm_w.is_contiguous(), "norm_w: [128] fp32")
    _require(head_scale is None or (head_scale.dtype == torch.float32 and head_scale.numel() == K // 128),
             "head_scale: [K / 128] fp32")
    _require(W.dim() == 2 and W.dtype == torch.int8 and W.shape[1] == K, "W: [N, K] int8")
    N = W.shape[0]
    _require(y.dtype == torch.float32 and y.dim() == 2 and y.shape[0] == M and y.shape[1] == N and y.stride(1) == 1,
             "y: [M, N] fp32")
    fmt = _weight_format(W, w_scale, N, K)
    st = _lib.lib().q35_gemv_gated_norm(_ptr(o), o.stride(0), _ptr(z), z.stride(0), _ptr(norm_w), _ptr(head_scale),
                                        float(eps), _ptr(W), fmt, _ptr(w_scale), _ptr(y), y.stride(0), M, N, K,
                                        int(epilogue), _stream(o))
    check(st, "q35_gemv_gated_norm")


def _swiglu_push_impl(gu, pushes, T, cap=None):
    _on_gpu(gu, pushes)
    _require(gu.dtype == torch.float32 and gu.shape[-1] % 2 == 0, "gu: [..., 2 I] fp32")
    I = gu.shape[-1] // 2
    M = gu.numel() // (2 * I)
    a = torch.empty(*gu.shape[:-1], I, dtype=torch.float32, device=gu.device)
    cp, ldc, ldcr = _cap_args(cap, M, int(T), I, gu.device)
    st = _lib.lib().q35_swiglu_push(_ptr(gu), _ptr(a), M, I, _ptr(pushes), _pushes_check(pushes), int(T), cp, ldc,
                                    ldcr, _stream(gu))
    check(st, "q35_swiglu_push")
    return a


def _add_rmsnorm_impl(x, y, w, eps, split=False):
    _on_gpu(x, y, w)
    _require(x.dtype == torch.float32 and w.dtype == torch.float32, "x, w fp32")
    H = x.shape[-1]
    _require(w.numel() == H and (y is None or (y.shape == x.shape and y.dtype == torch.float32)),
             "w: [H]; y like x")
    M = x.numel() // H
    h = torch.empty_like(x, dtype=torch.int32 if split else torch.float32)
    fn = "q35_add_rmsnorm_split" if split else "q35_add_rmsnorm"
    st = getattr(_lib.lib(), fn)(_ptr(x), H, _ptr(y), H, _ptr(w), _ptr(h), H, M, H, float(eps), _stream(x))
    check(st, fn)
    return h


def _add_rmsnorm_split_impl(x, y, w, eps):
    return _add_rmsnorm_impl(x, y, w, eps, split=True)


def _argmax_rows_impl(x, idx):
    _on_gpu(x, idx)
    _require(x.dtype == torch.float32 and x.dim() == 2 and x.stride(1) == 1, "x: [rows, n] fp32, rows dense")
    _require(idx.dtype == torch.int32 and idx.is_contiguous() and idx.numel() == x.shape[0], "idx: [rows] int32")
    st = _lib.lib().q35_argmax_rows(_ptr(x), x.stride(0), x.shape[0], x.shape[1], _ptr(idx), None, _stream(x))
    check(st, "q35_argmax_rows")


def _no_cpu(name):
    def f(*args, **kwargs):
        raise Q35Error(f"q35hip: q35::{name} needs HIP device tensors; the product has no CPU path")
    return f


for _name, _impl in [("gdn_recurrent", _gdn_recurrent_impl), ("gdn_decode_step_", _gdn_decode_step_impl),
                     ("gdn_chunk_prefill", _gdn_chunk_impl), ("gated_attn_prefill", _attn_prefill_impl),
                     ("gated_attn_prefill_cached", _attn_prefill_cached_impl),
                     ("gated_attn_decode", _attn_decode_impl), ("resid_add_rows_", _resid_add_impl),
                     ("gated_attn_decode_proj", _attn_decode_proj_impl),
                     ("gated_attn_prefill_proj", _attn_prefill_proj_impl),
                     ("gated_attn_prefill_cached_proj", _attn_prefill_cached_proj_impl),
                     ("gdn_conv", _gdn_conv_impl), ("gated_rmsnorm", _gated_rmsnorm_impl), ("gated_rmsnorm_split", _gated_rmsnorm_split_impl),
                     ("gdn_decode_fused_", _gdn_decode_fused_impl),
                     ("attn_prep", _attn_prep_impl), ("gemv_", _gemv_impl), ("swiglu_push", _swiglu_push_impl),
                     ("gemm_q8_", _gemm_q8_impl),
                     ("add_rmsnorm_", _add_rmsnorm_impl), ("add_rmsnorm_split_", _add_rmsnorm_split_impl),
                     ("argmax_rows_", _argmax_rows_impl),
                     ("gemv_norm_", _gemv_norm_impl), ("gdn_decode_sliced_", _gdn_decode_sliced_impl),
                     ("gemv_norm_argmax_", _gemv_norm_argmax_impl),
                     ("gdn_chunk_prefill_conv_", _gdn_chunk_prefill_conv_impl),
                     ("gemv_norm_conv_", _gemv_norm_conv_impl), ("gemv_gated_norm_", _gemv_gated_norm_impl)]:
    _LIB.impl(_name, _impl, "CUDA")
    _LIB.impl(_name, _no_cpu(_name), "CPU")


# Meta (shape-only) kernels
def _meta_gdn(q, k, v, g, beta, initial_state, *rest):
    B, T, Hk, Dk = q.shape
    H, Dv = v.shape[2], v.shape[3]
    return torch.empty_like(v), v.new_empty(B, H, Dk, Dv, dtype=torch.float32)


_LIB.impl("gdn_recurrent", _meta_gdn, "Meta")
_LIB.impl("gdn_chunk_prefill", _meta_gdn, "Meta")
_LIB.impl("gdn_decode_step_", lambda q, k, v, g, beta, state, scale, l2: torch.empty_like(v), "Meta")
_LIB.impl("gated_attn_prefill",
          lambda q, k, v, gate, cos, sin, pos0, scale: q.new_empty(q.shape[0], q.shape[1], q.shape[2] * q.shape[3]),
          "Meta")
_LIB.impl("gated_attn_decode",
          lambda q, kc, vc, gate, cl, cos, sin, scale, splits, f32_out=False:
          q.new_empty(q.shape[0], q.shape[1] * q.shape[2], dtype=torch.float32 if f32_out else q.dtype),
          "Meta")
_LIB.impl("gated_attn_decode_proj",
          lambda y, qn, kn, eps, kc, vc, pos, cos, sin, Hq, scale, splits, f32_out=False:
          y.new_empty(y.shape[0], Hq * kc.shape[3], dtype=torch.float32 if f32_out else torch.bfloat16),
          "Meta")
_LIB.impl("gated_attn_prefill_proj",
          lambda y, qn, kn, eps, kc, vc, pos0, cos, sin, Hq, scale:
          y.new_empty(y.shape[0], y.shape[1], Hq * kc.shape[3], dtype=torch.bfloat16),
          "Meta")
_LIB.impl("gated_attn_prefill_cached_proj",
          lambda y, qn, kn, eps, kc, vc, pos, cos, sin, Hq, scale:
          y.new_empty(y.shape[0], y.shape[1], Hq * kc.shape[3], dtype=torch.bfloat16),
          "Meta")
_LIB.impl("resid_add_rows_", lambda x, vecs, vor: None, "Meta")
_LIB.impl("gdn_decode_fused_", lambda y, cw, cb, cs, Al, dt, bo, ao, zo, st, nw, hs, eps, sc:
          y.new_empty(y.shape[0], st.shape[1] * st.shape[2]), "Meta")
_LIB.impl("gated_attn_prefill_cached",
          lambda q, kc, vc, gate, pos, cos, sin, scale: q.new_empty(q.shape[0], q.shape[1], q.shape[2] * q.shape[3]),
          "Meta")
_LIB.impl("argmax_rows_", lambda x, idx: None, "Meta")
_LIB.impl("gemv_norm_", lambda x, xa, xo, nw, eps, W, ws, y, e, pushes, T, cap=None: None, "Meta")
_LIB.impl("gemv_norm_argmax_", lambda x, xa, xo, nw, eps, W, ws, y, slots, idx: None, "Meta")
_LIB.impl("gdn_chunk_prefill_conv_", lambda y, cw, cb, cs, Al, dt, bo, ao, st, Hk, sc:
          y.new_empty(y.shape[0], y.shape[1], st.shape[1], st.shape[3]), "Meta")
_LIB.impl("gdn_decode_sliced_", lambda y, Al, dt, bo, ao, st, sc: y.new_empty(y.shape[0], st.shape[1] * st.shape[2]),
          "Meta")
_LIB.impl("gemv_norm_conv_", lambda x, xa, xo, nw, eps, W, ws, y, cw, cb, cs: None, "Meta")
_LIB.impl("gemv_gated_norm_", lambda o, z, nw, hs, eps, W, ws, y, e: None, "Meta")
_LIB.impl("gemv_", lambda x, W, ws, y, e, pushes, T, cap=None: None, "Meta")
_LIB.impl("gemm_q8_", lambda x, W, ws, y, e, pushes, T, cap=None: None, "Meta")
_LIB.impl("swiglu_push", lambda gu, pushes, T, cap=None: gu.new_empty(*gu.shape[:-1], gu.shape[-1] // 2),
          "Meta")
_LIB.impl("add_rmsnorm_", lambda x, y, w, eps: torch.empty_like(x), "Meta")
_LIB.impl("add_rmsnorm_split_", lambda x, y, w, eps: torch.empty_like(x, dtype=torch.int32), "Meta")
_LIB.impl("gated_rmsnorm", lambda o, z, w, hs, eps: o.new_empty(*o.shape[:-2], o.shape[-2] * o.shape[-1]), "Meta")
_LIB.impl("gated_rmsnorm_split", lambda o, z, w, hs, eps: o.new_empty(*o.shape[:-2], o.shape[-2] * o.shape[-1],
                                                                      dtype=torch.int32), "Meta")


def _meta_gdn_conv(y, conv_w, conv_bias, conv_state, A_log, dt_bias, b_off, a_off, Hk, dk, Hv, dv, bf16_out):
    B, T = y.shape[0], y.shape[1]
    dt = torch.bfloat16 if bf16_out else torch.float32
    q = y.new_empty(B, T, Hk, dk, dtype=dt)
    g = y.new_empty(B, T, Hv, dtype=torch.float32)
    return q, torch.empty_like(q), y.new_empty(B, T, Hv, dv, dtype=dt), g, torch.empty_like(g)


def _meta_attn_prep(y, q_norm_w, k_norm_w, eps, cos, sin, pos, k_cache, v_cache, Hq, Hkv, want_kv):
    B, T = y.shape[0], y.shape[1]
    D = k_cache.shape[3]
    q = y.new_empty(B, T, Hq, D, dtype=torch.bfloat16)
    gate = y.new_empty(B, T, Hq * D, dtype=torch.bfloat16)
    k = y.new_empty(B, T, Hkv, D, dtype=torch.bfloat16) if want_kv else y.new_empty(0, dtype=torch.bfloat16)
    return q, gate, k, torch.empty_like(k)


_LIB.impl("gdn_conv", _meta_gdn_conv, "Meta")
_LIB.impl("attn_prep", _meta_attn_prep, "Meta")


# ---------------------------------------------------------------- Python entry points (reference signatures)
def _hf_args(query, key, value, g, beta, initial_state):
    """HF passes q / k / v as strided views of the conv output (HF:482-502) and beta in the model dtype: make them
    dense, with g, beta and the state in fp32."""
    query, key, value = query.contiguous(), key.contiguous(), value.contiguous()
    if value.dtype != query.dtype:
        value = value.to(query.dtype)
    g, beta = g.float().contiguous(), beta.float().contiguous()
    if initial_state is not None:
        initial_state = initial_state.float().contiguous()
    return query, key, value, g, beta, initial_state


def recurrent_gated_delta_rule(query, key, value, g, beta, initial_state=None, output_final_state=False,
                               use_qk_l2norm_in_kernel=False, scale=None, **kwargs):
    """Drop-in for torch_recurrent_gated_delta_rule (HF:331-380): [B, T, H, D] layouts, returns
    (o in the input dtype, final fp32 state or None)."""
    scale = 1.0 / math.sqrt(key.shape[-1]) if scale is None else scale
    query, key, value, g, beta, initial_state = _hf_args(query, key, value, g, beta, initial_state)
    o, S = torch.ops.q35.gdn_recurrent(query, key, value, g, beta, initial_state, scale,
                                       bool(use_qk_l2norm_in_kernel))
    return o, (S if output_final_state else None)


def chunk_gated_delta_rule(query, key, value, g, beta, chunk_size=64, initial_state=None, output_final_state=False,
                           use_qk_l2norm_in_kernel=False, scale=None, **kwargs):
    """Drop-in for torch_chunk_gated_delta_rule (HF:249-327); chunk_size must be 64."""
    scale = 1.0 / math.sqrt(key.shape[-1]) if scale is None else scale
    query, key, value, g, beta, initial_state = _hf_args(query, key, value, g, beta, initial_state)
    o, S = torch.ops.q35.gdn_chunk_prefill(query, key, value, g, beta, initial_state, int(chunk_size), scale,
                                           bool(use_qk_l2norm_in_kernel))
    return o, (S if output_final_state else None)


def gdn_decode_step_(query, key, value, g, beta, state, use_qk_l2norm_in_kernel=True, scale=None):
    """One (or more) token(s) of the recurrence with the fp32 state updated in place; returns o."""
    scale = 1.0 / math.sqrt(key.shape[-1]) if scale is None else scale
    return torch.ops.q35.gdn_decode_step_(query, key, value, g, beta, state, scale, bool(use_qk_l2norm_in_kernel))


def gated_attention_prefill(q, k, v, gate, cos, sin, pos0=0, scale=None):
    """Causal gated GQA attention with partial RoPE (q: [B, T, Hq, D]; k, v: [B, T, Hkv, D]; gate: [B, T, Hq*D];
    cos/sin: [P, rot/2] fp32 by position). Returns [B, T, Hq*D] bf16."""
    scale = q.shape[-1] ** -0.5 if scale is None else scale
    return torch.ops.q35.gated_attn_prefill(q, k, v, gate, cos, sin, int(pos0), float(scale))


def gated_attention_prefill_cached(q, k_cache, v_cache, gate, pos, cos, sin, scale=None):
    """Causal gated GQA attention of T new tokens per row over a bf16 KV cache that already holds them (the
    reference's multi-token attention, engine/kernels_qwen35.js:90: token t of row b sits at position pos[b] + t and
    attends to cache keys 0 .. pos[b] + t). q: [B, T, Hq, D] bf16, not rotated (rotated here at its position);
    caches [B, Hkv, max_len, D] with rotated keys, max_len a multiple of 64; pos: [B] int32 on the device (clamped to
    0 .. max_len - T); gate [B, T, Hq * D]. Returns [B, T, Hq * D] bf16."""
    scale = q.shape[-1] ** -0.5 if scale is None else scale
    return torch.ops.q35.gated_attn_prefill_cached(q, k_cache, v_cache, gate, pos, cos, sin, float(scale))


def gated_attention_decode(q, k_cache, v_cache, gate, cache_len, cos, sin, scale=None, splits=0,
                           out_dtype=torch.bfloat16):
    """One new token per row over a bf16 KV cache [B, Hkv, max_len, D]; q rotated at position cache_len - 1. The
    output [B, Hq * D] is bf16, or fp32 with out_dtype=torch.float32 (written so by the merge kernel itself)."""
    scale = q.shape[-1] ** -0.5 if scale is None else scale
    return torch.ops.q35.gated_attn_decode(q, k_cache, v_cache, gate, cache_len, cos, sin, float(scale), int(splits),
                                           out_dtype == torch.float32)


def gated_attention_decode_proj(y, q_norm_w, k_norm_w, k_cache, v_cache, pos, cos, sin, *, num_heads, eps=1e-6,
                                scale=None, splits=0, out_dtype=torch.bfloat16):
    """The attention decode step from the fused projection output y [B, W] (or [B, 1, W]) fp32 of one token per row
    ([q | gate] per head, then k, then v; engine/kernels_qwen35.js:18-123 attnPrep + attention): q and k normalised
    with (1 + w) and rotated at position pos[b] ([B] int32 on the device), the token's key and value appended to the
    bf16 caches at pos[b], attention over cache keys 0 .. pos[b], sigmoid gate. Returns [B, num_heads * D] bf16, or
    fp32 with out_dtype=torch.float32."""
    D = k_cache.shape[3]
    scale = D ** -0.5 if scale is None else scale
    return torch.ops.q35.gated_attn_decode_proj(y, q_norm_w.float().contiguous(), k_norm_w.float().contiguous(),
                                                float(eps), k_cache, v_cache, pos, cos, sin, int(num_heads),
                                                float(scale), int(splits), out_dtype == torch.float32)


def gated_attention_prefill_proj(y, q_norm_w, k_norm_w, k_cache, v_cache, cos, sin, *, num_heads, pos0=0, eps=1e-6,
                                 scale=None):
    """Causal gated attention of the call's own T tokens per row from the fused projection output y [B, T, W] fp32
    ([q | gate] per head, then k, then v; engine/kernels_qwen35.js:18-123 attnPrep + attention at positions
    pos0 .. pos0 + T - 1): q and k normalised with (1 + w) and rotated, the keys and values appended to the bf16
    caches [B, Hkv, max_len, D] at those positions, sigmoid gate. Returns [B, T, num_heads * D] bf16."""
    D = k_cache.shape[3]
    scale = D ** -0.5 if scale is None else scale
    return torch.ops.q35.gated_attn_prefill_proj(y, q_norm_w.float().contiguous(), k_norm_w.float().contiguous(),
                                                 float(eps), k_cache, v_cache, int(pos0), cos, sin, int(num_heads),
                                                 float(scale))


def gated_attention_prefill_cached_proj(y, q_norm_w, k_norm_w, k_cache, v_cache, pos, cos, sin, *, num_heads,
                                        eps=1e-6, scale=None):
    """T new tokens per row over the bf16 KV cache from their fused projection output y [B, T, W] fp32 (the
    reference's multi-token attention, engine/kernels_qwen35.js:18-123 attnPrep + attention, with token t of row b at
    position pos[b] + t, pos: [B] int32 on the device, clamped to 0 .. max_len - T): q and k normalised with (1 + w)
    and rotated, the tokens' keys and values appended to the caches, attention over cache keys 0 .. pos[b] + t,
    sigmoid gate; max_len a multiple of 64. Returns [B, T, num_heads * D] bf16."""
    D = k_cache.shape[3]
    scale = D ** -0.5 if scale is None else scale
    return torch.ops.q35.gated_attn_prefill_cached_proj(y, q_norm_w.float().contiguous(),
                                                        k_norm_w.float().contiguous(), float(eps), k_cache, v_cache,
                                                        pos, cos, sin, int(num_heads), float(scale))


def residual_steer_add_(x, vecs, vec_of_row=None):
    """x[r, t, :] += vecs[vec_of_row[r]] in place (negative index: no vector; None: min(r, nvec - 1))."""
    torch.ops.q35.resid_add_rows_(x, vecs, vec_of_row)
    return x


def gdn_conv(y, conv_w, conv_state, A_log, dt_bias, *, num_k_heads, head_k_dim, num_v_heads, head_v_dim, b_off, a_off,
             conv_bias=None, out_dtype=torch.float32):
    """Gated DeltaNet front end (HF:454-499; engine/kernels_qwen35.js:127-178, :226-229) over the fused projection
    output y [B, T, W]: returns (q, k [B, T, Hk, dk], v [B, T, Hv, dv] in out_dtype, g, beta [B, T, Hv] fp32) and
    advances conv_state [B, K - 1, C] in place."""
    w = conv_w.reshape(conv_w.shape[0], conv_w.shape[-1])
    return torch.ops.q35.gdn_conv(y, w.float().contiguous(), conv_bias, conv_state, A_log.float().contiguous(),
                                  dt_bias.float().contiguous(), int(b_off), int(a_off), int(num_k_heads),
                                  int(head_k_dim), int(num_v_heads), int(head_v_dim), out_dtype == torch.bfloat16)


def gdn_decode_fused_(y, conv_w, conv_state, A_log, dt_bias, state, norm_w, *, b_off, a_off, z_off, head_scale=None,
                      conv_bias=None, eps=1e-6, scale=None):
    """One Gated DeltaNet decode step after the input projection, in one launch (gdn_conv for one token, the
    recurrent rule with l2norm on the state, gated_rmsnorm; HF:454-543 for a cached token): y [B, W] fp32 rows of
    the fused projection, conv_state [B, K - 1, C] and state [B, H, d, d] advanced in place (Hk = Hv = H,
    dk = dv = d = 128). Returns the gated-normed output [B, H * d] fp32."""
    H, d = state.shape[1], state.shape[2]
    w = conv_w.reshape(conv_w.shape[0], conv_w.shape[-1])
    return torch.ops.q35.gdn_decode_fused_(y, w.float().contiguous(), conv_bias, conv_state,
                                           A_log.float().contiguous(), dt_bias.float().contiguous(), int(b_off),
                                           int(a_off), int(z_off), state, norm_w.float().contiguous(), head_scale,
                                           float(eps), float(d ** -0.5 if scale is None else scale))


def gdn_chunk_prefill_conv_(y, conv_w, conv_state, A_log, dt_bias, state, *, num_k_heads, b_off, a_off,
                            conv_bias=None, scale=None):
    """A Gated DeltaNet layer's multi-token call from its fused projection output y [B, T, W] fp32 up to the gated
    norm: gdn_conv (fp32) then chunk_gated_delta_rule (l2norm on) in one kernel pair, the conv + SiLU and the gate
    terms in the chunk kernel's load phase (HF:454-530). conv_state [B, 3, C] and state [B, H, d, d] (d = 128; the
    initial state, then the final one) are advanced in place; returns o [B, T, H, d] fp32. The conv kernel size must
    be 4."""
    d = state.shape[-1]
    w = conv_w.reshape(conv_w.shape[0], conv_w.shape[-1])
    return torch.ops.q35.gdn_chunk_prefill_conv_(y, w.float().contiguous(), conv_bias, conv_state,
                                                 A_log.float().contiguous(), dt_bias.float().contiguous(), int(b_off),
                                                 int(a_off), state, int(num_k_heads),
                                                 float(d ** -0.5 if scale is None else scale))


def gdn_decode_sliced_(y, A_log, dt_bias, state, *, b_off, a_off, scale=None):
    """The recurrent part of a Gated DeltaNet decode step (HF:454-543 for a cached token, from the recurrent rule on)
    over projection rows y [B, W] fp32 whose q|k|v channels already went through the causal conv + SiLU
    (gemv(..., conv=...)): state [B, H, d, d] advanced in place (Hk = Hv = H, d = 128). Returns the raw output
    o [B, H * d] fp32, before the gated RMSNorm (gemv_gated_norm applies it)."""
    d = state.shape[2]
    return torch.ops.q35.gdn_decode_sliced_(y, A_log.float().contiguous(), dt_bias.float().contiguous(), int(b_off),
                                            int(a_off), state, float(d ** -0.5 if scale is None else scale))


def gemv_gated_norm(o, z, norm_w, W, w_scale, out, *, head_scale=None, eps=1e-6, epilogue="store"):
    """out (=, or += for epilogue "add") gated_rmsnorm(o, z) @ W^T s for M <= 8 rows: the GDN layer's output norm
    (HF:168-184) applied per head of 128 while the product stages o (q35_gemv_gated_norm). W int8 [N, K] with
    w_scale [N, K / 128] or [N]; o [M, K], z [M, >= K] fp32."""
    torch.ops.q35.gemv_gated_norm_(o, z, norm_w.float().contiguous(), head_scale, float(eps), W, w_scale, out,
                                   _EPI[epilogue])
    return out


def gated_rmsnorm(o, z, w, head_scale=None, eps=1e-6, split=False):
    """Qwen3_5RMSNormGated (HF:168-184) per (token, head) with the engine's optional per-head scale
    (engine/kernels_qwen35.js:243): o [..., Hv, dv], z [..., Hv * dv] fp32 (rows may be strided) -> [..., Hv * dv].
    split=True (fp32 o): the int32 words of the result in the int8 GEMM's split layout (split_activations)."""
    if split:
        return torch.ops.q35.gated_rmsnorm_split(o, z, w.float().contiguous(), head_scale, float(eps))
    return torch.ops.q35.gated_rmsnorm(o, z, w.float().contiguous(), head_scale, float(eps))


def attn_prep(y, q_norm_w, k_norm_w, cos, sin, pos, k_cache, v_cache, *, num_heads, num_kv_heads, eps=1e-6,
              want_kv=True):
    """Attention front end (HF:667-680; engine/kernels_qwen35.js:18-69) over the fused projection output y: returns
    (q [B, T, Hq, D], gate [B, T, Hq * D], k, v [B, T, Hkv, D]) in bf16, q and k RMS-normalised with (1 + w) and not
    rotated, and writes rotated keys and values into the caches at positions pos[b] + t (pos: [B] int32 device)."""
    return torch.ops.q35.attn_prep(y, q_norm_w.float().contiguous(), k_norm_w.float().contiguous(), float(eps), cos,
                                   sin, pos, k_cache, v_cache, int(num_heads), int(num_kv_heads), bool(want_kv))


def pack_pushes(pushes, device):
    """Neuron pushes [(neuron or None for every neuron, "add" | "mul", [value per row, up to 4])] as the [n, 6] int32
    records of the C ABI (engine/model.js:412-423: missing row values are 0 for add and 1 for mul)."""
    import struct
    rec = []
    for neuron, mode, vals in pushes:
        m = {"add": 0, "mul": 1}[mode]
        v = [float(x) for x in vals] + [1.0 if m else 0.0] * (4 - len(vals))
        rec.append([-1 if neuron is None else int(neuron), m] + [struct.unpack("<i", struct.pack("<f", x))[0]
                                                                 for x in v[:4]])
    return torch.tensor(rec, dtype=torch.int32).reshape(-1, 6).to(device)


def gemv(x, W, w_scale=None, out=None, epilogue="store", pushes=None, T=1, prenorm=None, conv=None, capture=None):
    """y[m, n] = sum_k x[m, k] W[n, k] s(n, k) for M <= 8 rows (decode): W int8 with scales w_scale [N, K / 128]
    (one per group of 128 inputs, the engine's q8 format) or [N] (one per row), or fp32 W (w_scale None).
    epilogue "store" writes out, "add" accumulates into out (a residual add; products with few output rows split K
    and add with fp32 atomics, so the last bits may vary between runs), "add_fixed" accumulates with every output
    summed in one fixed order (repeatable bits), "swiglu" treats W's rows as interleaved (gate, up) pairs and writes
    silu(gate) * up with the neuron pushes (pack_pushes) applied.
    prenorm = (x_add, norm_w, eps, x_out): x is then a residual; the product takes the RMSNorm (1 + w) of
    s = x + x_add (x_add may be None), and s is written to x_out when it is not None (q35_gemv_norm).
    conv = (conv_w [C, K], conv_bias or None, conv_state [M, K - 1, C]), with prenorm and the store epilogue: outputs
    0 .. C - 1 go through the GDN causal conv + SiLU and conv_state advances in place (q35_gemv_norm_conv).
    capture (SwiGLU only): an fp32 view [rows, T, I] or [M, I] (unit neuron stride) that also receives the
    activations after the pushes (the engine's MLP capture hook, engine/model.js:9, :451-453)."""
    e = _EPI[epilogue]
    if out is None:
        N = W.shape[0] // 2 if e == 2 else W.shape[0]
        out = torch.empty(x.shape[0], N, dtype=torch.float32, device=x.device)
    if conv is not None:
        _require(prenorm is not None and e == 0, "the conv epilogue runs with prenorm and the store epilogue")
        x_add, norm_w, eps, x_out = prenorm
        cw, cb, cs = conv
        torch.ops.q35.gemv_norm_conv_(x, x_add, x_out, norm_w, float(eps), W, w_scale, out,
                                      cw.reshape(cw.shape[0], cw.shape[-1]).float().contiguous(), cb, cs)
        return out
    if prenorm is None:
        torch.ops.q35.gemv_(x, W, w_scale, out, e, pushes, int(T), capture)
    else:
        x_add, norm_w, eps, x_out = prenorm
        torch.ops.q35.gemv_norm_(x, x_add, x_out, norm_w, float(eps), W, w_scale, out, e, pushes, int(T), capture)
    return out


def gemm_q8(x, W, w_scale, out=None, epilogue="store", pushes=None, T=1, split_out=False, capture=None):
    """y[m, n] = sum_k x[m, k] W[n, k] s(n, k) over many rows (the prefill projections): x [M, K] fp32, W [N, K]
    int8 with scales w_scale [N, K / 128] (per group of 128 inputs) or [N] (per row), K a multiple of 64 (128 with
    group scales); fp32-accurate (bf16 MFMA on a hi + lo split of x). epilogue "store" writes out, "add"
    accumulates into out, "swiglu" treats W's rows as interleaved (gate, up) pairs and writes
    silu(gate) * up with the neuron pushes (pack_pushes) applied, out [M, N / 2]. x may also be the int32 words of
    activations already split (add_rmsnorm_(..., split=True), split_activations): the same product, bitwise, without
    the split in the kernel; or bf16 (the lo products skipped: the product of x.float() bitwise where that runs the register-staged
    kernel, N < 2048 or K > 2048, and to fp32 rounding on the wide shapes). split_out=True (SwiGLU only) writes out as the int32 words of the split layout, the
    input of the next gemm_q8. capture: as for gemv (the fp32 activations, whatever the layout of out). Returns out."""
    e = _EPI[epilogue]
    if split_out:
        if e != 2:
            raise ValueError("gemm_q8: split_out is a form of the SwiGLU epilogue")
        e = 3
    x = x if x.stride(-1) == 1 else x.contiguous()
    if out is None:
        N = W.shape[0] // 2 if e in (2, 3) else W.shape[0]
        out = torch.empty(x.shape[0], N, dtype=torch.int32 if e == 3 else torch.float32, device=x.device)
    torch.ops.q35.gemm_q8_(x, W, w_scale, out, e, pushes, int(T), capture)
    return out


def swiglu_push(gu, pushes=None, T=1, capture=None):
    """silu(gate) * up over a [..., 2 I] ([gate | up]) projection with the neuron pushes applied (the hook point of
    engine/kernels_qwen35.js:250-279); capture as for gemv."""
    return torch.ops.q35.swiglu_push(gu, pushes, int(T), capture)


def gemv_norm_argmax(x, W, w_scale, prenorm, slots, out=None, idx=None):
    """The store GEMV behind the RMSNorm prologue (gemv with prenorm = (x_add, norm_w, eps, x_out)) with each row's
    argmax of the result folded in (q35_gemv_norm_argmax: the greedy pick over the LM head's logits, lowest index on
    ties as argmax_rows). slots: [M] int64 device buffer holding zeros (each call leaves it zero). Returns (y [M, N]
    fp32, idx [M] int32)."""
    x_add, norm_w, eps, x_out = prenorm
    if out is None:
        out = torch.empty(x.shape[0], W.shape[0], dtype=torch.float32, device=x.device)
    if idx is None:
        idx = torch.empty(x.shape[0], dtype=torch.int32, device=x.device)
    torch.ops.q35.gemv_norm_argmax_(x, x_add, x_out, norm_w, float(eps), W, w_scale, out, slots, idx)
    return out, idx


def argmax_rows(x, out=None):
    """Per-row argmax of x [rows, n] fp32 (lowest index on ties, as torch.argmax and the engine's WGSL argmax,
    engine/kernels.js:260-283) into out ([rows] int32, allocated when None). Returns out."""
    x = x if x.stride(-1) == 1 else x.contiguous()
    if out is None:
        out = torch.empty(x.shape[0], dtype=torch.int32, device=x.device)
    torch.ops.q35.argmax_rows_(x, out)
    return out


def add_rmsnorm_(x, y, w, eps=1e-6, split=False):
    """x += y in place (y None: no add), then return x * rsqrt(mean x^2 + eps) * (1 + w) (Qwen3_5RMSNorm, HF:720-734),
    fp32, x and y dense [..., H]. split=True returns the normed rows as int32 words in the int8 GEMM's split layout
    (split_activations of the fp32 result, H a multiple of 8), which gemm_q8 reads without splitting them again."""
    if split:
        return torch.ops.q35.add_rmsnorm_split_(x, y, w.float().contiguous(), float(eps))
    return torch.ops.q35.add_rmsnorm_(x, y, w.float().contiguous(), float(eps))


def split_activations(x):
    """fp32 rows [..., K] (K a multiple of 8) in the int8 GEMM's split layout, as int32 words of the same shape: each
    value as hi = bf16(x) and lo = bf16(x - hi) (round to nearest even), each group of 8 inputs as its 8 hi parts
    followed by its 8 lo parts. Torch ops on any device (the layout's definition; the product path produces it in
    add_rmsnorm_(..., split=True))."""
    if x.dtype != torch.float32 or x.shape[-1] % 8:
        raise ValueError("split_activations: fp32 rows with a multiple of 8 inputs")
    hi = x.to(torch.bfloat16)
    lo = (x - hi.float()).to(torch.bfloat16)
    g = x.shape[:-1] + (x.shape[-1] // 8, 8)
    return torch.cat([hi.reshape(g), lo.reshape(g)], dim=-1).reshape(x.shape[:-1] + (2 * x.shape[-1],)).contiguous() \
        .view(torch.int32)
