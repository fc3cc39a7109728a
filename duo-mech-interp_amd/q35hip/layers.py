"""Per-layer forward functions of the Qwen3.5 hybrid decoder, running the hot path on the q35:: HIP ops.

    gated_deltanet_layer(x, p, conv_state, rec_state, head_scale=None) -> y
    gated_attention_layer(x, p, k_cache, v_cache, pos) -> y
    residual_steer_add(x, vecs, rows) -> x

`p` holds one layer's weights under HF's parameter names (transformers 5.15.0 models/qwen3_5/modeling_qwen3_5.py,
HF:426-429 and HF:641-654; the engine's names at engine/model.js:89-112 map one to one):
  Gated DeltaNet   in_proj_qkv [C, H], in_proj_z [Hv*dv, H], in_proj_b [Hv, H], in_proj_a [Hv, H],
                   conv1d [C, K] (HF's [C, 1, K] is accepted), A_log [Hv], dt_bias [Hv], norm [dv], out_proj [H, Hv*dv]
  gated attention  q_proj [Hq*2*D, H] (per head [q | gate], HF:667-670), k_proj [Hkv*D, H], v_proj [Hkv*D, H],
                   o_proj [H, Hq*D], q_norm [D], k_norm [D]
States are caller-owned device tensors mutated in place, as the engine's buffers are (engine/model.js:308-342):
conv_state [B, K-1, C] fp32 (the last K-1 conv inputs, oldest first, engine/model.js:333), rec_state [B, Hv, dk, dv]
fp32, k_cache / v_cache [B, Hkv, max_len, D] bf16 holding rotated keys and values by position.

Any weight may also come as int8 with fp32 scales ("<name>.q" / "<name>.s", one scale per group of 128 inputs as the
engine stores every linear, engine/model.js:3-5 and engine/kernels.js:15-47, or one per row; "<name>" then holds the
dequantised values). The input projections are stacked into one weight per mixer (cached in p under "_in_fused", with
"_in_fused.q" / ".s"). A projection over at most 8 rows (decode) is a HIP GEMV, over more rows the HIP int8 GEMM, on
the int8 weights when present; without them a torch GEMM on the fp32 weight. Every other
step is a HIP kernel: the GDN front end (causal conv + SiLU + gate terms), the delta rule, the gated RMSNorm,
the attention front end (q/k norms, q/gate split, KV-cache update), the attention itself and the steering add.
Nothing here falls back to a CPU path: the ops raise on CPU tensors and when the library is missing.
"""
import math

import torch

from . import ops

_ROPE_CACHE = {}


def rope_tables(n_pos, rot, theta, device):
    """cos / sin [n_pos, rot/2] fp32 of angle pos * theta^(-2j/rot) (HF:105-125 inv_freq in fp32, then the fp32
    product by position), cached per (n_pos, rot, theta, device)."""
    key = (int(n_pos), int(rot), float(theta), str(device))
    t = _ROPE_CACHE.get(key)
    if t is None:
        inv_freq = 1.0 / (theta ** (torch.arange(0, rot, 2, dtype=torch.int64).to(torch.float) / rot))
        ang = torch.arange(n_pos, dtype=torch.float32)[:, None] * inv_freq[None, :]
        t = (ang.cos().contiguous().to(device), ang.sin().contiguous().to(device))
        _ROPE_CACHE[key] = t
    return t


def rmsnorm_1p(x, w, eps=1e-6):
    """x * rsqrt(mean x^2 + eps) * (1 + w) in fp32 (HF:720-734; engine/kernels_qwen35.js:46-47)."""
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * (1.0 + w.float())).to(x.dtype)


def gated_deltanet_layer(x, p, conv_state, rec_state, head_scale=None, *, num_k_heads=None, head_k_dim=None,
                         eps=1e-6, prefill="chunk", prenorm=None, residual=None, fixed_order=False):
    """Gated DeltaNet mixer of one decoder layer (Qwen3_5GatedDeltaNet.forward, HF:432-543; the WGSL conv + delta
    kernels, engine/kernels_qwen35.js:127-247). x: [B, T, H] fp32 (the input-normed residual). A call with T == 1
    is one recurrent decode step (HF:505-517). T > 1 runs from rec_state either the chunked prefill (HF:518-530;
    prefill="chunk": products at the precision of x, fp32 for fp32 x) or the token-serial fp32 recurrence
    (prefill="recurrent": as the WGSL engine runs prefill token by token, engine/kernels_qwen35.js:183-247). Both
    states are updated in place. head_scale: optional [Hv] per-head output scale applied after the gated norm
    (engine/kernels_qwen35.js:243). num_k_heads / head_k_dim default to the
    value heads / value head dim (the Qwen3.5 text models use Hk = Hv and dk = dv). prenorm: see linear() (x is then
    the residual and the layer's input norm runs inside the input projection). Returns y [B, T, H], or with
    residual [B, T, H] given, residual + y computed in place by the output projection (then returned). For T > 1,
    x may be the int32 words of the normed rows already split for the int8 GEMM (add_rmsnorm_(..., split=True);
    the layer must then have int8 input projections). fixed_order: the decode step's residual add sums every output
    in one fixed order (repeatable bits; see linear())."""
    if prefill not in ("chunk", "recurrent"):
        raise ValueError(f"gated_deltanet_layer: prefill must be 'chunk' or 'recurrent', not {prefill!r}")
    B, T, _ = x.shape
    Hv = p["A_log"].numel()
    dv = p["norm"].numel()
    Hk = Hv if num_k_heads is None else num_k_heads
    dk = dv if head_k_dim is None else head_k_dim
    C, Vd = 2 * Hk * dk + Hv * dv, Hv * dv
    # one GEMM for every projection of the token: y row = [qkv (C) | z (Vd) | b (Hv) | a (Hv)], the engine's fused
    # layout (engine/kernels_qwen35.js:129-131)
    w_in = gdn_in_weight(p)
    wq_in, ws_in = _q8(p, "_in_fused")
    wq_out, ws_out = _q8(p, "out_proj")
    if (T == 1 and Hk == Hv and dk == dv == 128 and x.dtype == torch.float32 and B <= 8 and x.shape[-1] % 256 == 0
            and Vd % 256 == 0 and wq_in is not None and wq_out is not None
            and wq_in.shape[0] <= ops.gemv_conv_max_n(B) and p["conv1d"].shape[-1] <= ops.GEMV_CONV_MAX_K):
        # decode step on int8 projections: the causal conv + SiLU in the input projection's epilogue (each channel
        # has one owner there, so its conv state advances in place), the recurrent rule over four blocks per head,
        # and the gated RMSNorm in the output projection's staging (the same arithmetic as the fused step below)
        y = linear(x, w_in, wq_in, ws_in, prenorm=prenorm, conv=(p["conv1d"], None, conv_state))
        y2 = y.view(B, y.shape[-1])
        o = ops.gdn_decode_sliced_(y2, p["A_log"], p["dt_bias"], rec_state, b_off=C + Vd, a_off=C + Vd + Hv)
        N = wq_out.shape[0]
        out = residual.view(B, N) if residual is not None else torch.empty(B, N, dtype=torch.float32, device=x.device)
        ops.gemv_gated_norm(o, y2[:, C:], p["norm"], wq_out, ws_out, out, head_scale=head_scale, eps=eps,
                            epilogue="store" if residual is None else ("add_fixed" if fixed_order else "add"))
        return residual if residual is not None else out.view(B, 1, N)
    y = linear(x, w_in, wq_in, ws_in, prenorm=prenorm)
    if T == 1 and Hk == Hv and dk == dv == 128 and x.dtype == torch.float32:
        # the decode step's conv, recurrent rule and gated norm in one launch (the same arithmetic as the three
        # kernels below)
        o = ops.gdn_decode_fused_(y.view(B, y.shape[-1]), p["conv1d"], conv_state, p["A_log"], p["dt_bias"],
                                  rec_state, p["norm"], b_off=C + Vd, a_off=C + Vd + Hv, z_off=C,
                                  head_scale=head_scale, eps=eps)
        return linear(o.view(B, 1, Vd), p["out_proj"], *_q8(p, "out_proj"), residual=residual,
                      fixed_order=fixed_order)
    if (T > 1 and prefill == "chunk" and _act_dtype(x) == torch.float32 and dk == dv == 128
            and p["conv1d"].shape[-1] == 4 and rec_state.is_contiguous()):
        # the conv + SiLU, l2 norms and gate terms in the chunk kernel's load phase (q, k, v, g, beta never written
        # out), the recurrent state advanced in place: the arithmetic of gdn_conv + chunk_gated_delta_rule below
        o = ops.gdn_chunk_prefill_conv_(y, p["conv1d"], conv_state, p["A_log"], p["dt_bias"], rec_state,
                                        num_k_heads=Hk, b_off=C + Vd, a_off=C + Vd + Hv)
    else:
        q, k, v, g, beta = ops.gdn_conv(y, p["conv1d"], conv_state, p["A_log"], p["dt_bias"], num_k_heads=Hk,
                                        head_k_dim=dk, num_v_heads=Hv, head_v_dim=dv, b_off=C + Vd,
                                        a_off=C + Vd + Hv, out_dtype=_act_dtype(x))
        if T == 1 or prefill == "recurrent":
            o = ops.gdn_decode_step_(q, k, v, g, beta, rec_state, use_qk_l2norm_in_kernel=True)
        else:
            o, S = ops.chunk_gated_delta_rule(q, k, v, g, beta, initial_state=rec_state, output_final_state=True,
                                              use_qk_l2norm_in_kernel=True)
            rec_state.copy_(S)
    # gated RMSNorm: plain w, norm before the silu(z) gate (HF:168-184; engine/kernels_qwen35.js:237-243)
    # (fp32 o before an int8 output projection: the result already split for the int8 GEMM)
    split = T > 1 and o.dtype == torch.float32 and wq_out is not None and Vd % 64 == 0
    o = ops.gated_rmsnorm(o, y[..., C:C + Vd], p["norm"], head_scale, eps, split=split)
    return linear(o, p["out_proj"], wq_out, ws_out, residual=residual)


def _act_dtype(x):
    """The value dtype of a layer input: fp32 for the int32 words of split activations."""
    return torch.float32 if x.dtype == torch.int32 else x.dtype


def prenorm_torch(x, prenorm):
    """The prenorm of linear() on torch ops: s = x + x_add (x_add may be None), copied to x_out when given; returns
    s * rsqrt(mean s^2 + eps) * (1 + w)."""
    x_add, nw, eps, x_out = prenorm
    s = x + x_add if x_add is not None else x.clone()
    if x_out is not None:
        x_out.copy_(s)
    return ops.add_rmsnorm_(s, None, nw, eps)


def linear(x, w, wq=None, ws=None, prenorm=None, residual=None, conv=None, fixed_order=False):
    """x [..., K] @ w[N, K]^T in fp32: the HIP GEMV for a few rows (decode), on the int8 weights wq with scales ws
    ([N, K / 128] per group or [N] per row; w their dequantised values) when given, else on w; for more rows the HIP
    int8 GEMM on wq (fp32-accurate) when given, else a torch GEMM on w. prenorm = (x_add, norm_w, eps, x_out): x is
    a residual and the product takes the RMSNorm (1 + norm_w) of x + x_add (x_add may be None), the sum being written
    to x_out when given (the decoder layer's add + norm, fused into the GEMV). residual [..., N]: the product is added
    into it in place (the decoder layer's residual add after its mixer) and residual is returned. conv =
    (conv_w, conv_bias, conv_state): the GEMV with prenorm runs the GDN causal conv + SiLU on the first
    conv_w.shape[0] outputs and advances conv_state (decode only: raises when the product is not a GEMV). x may be the
    int32 words of split activations (ops.split_activations) when wq is given: the int8 GEMM reads them as they are.
    fixed_order (with residual): the decode GEMV sums every output in one fixed order (the "add_fixed" epilogue:
    repeatable bits) instead of splitting K over blocks that add with atomics; the GEMM's sums are always in a fixed
    order."""
    K = x.shape[-1]
    M = x.numel() // K
    N = (wq if wq is not None else w).shape[0]
    out, epi = (None, "store") if residual is None else (residual.view(M, N), "add_fixed" if fixed_order else "add")
    if M <= 8 and K % 256 == 0 and x.dtype == torch.float32 and (wq is not None or w.dtype == torch.float32):
        xm = x.reshape(M, K).contiguous()
        pn = None
        if prenorm is not None:
            x_add, nw, eps, x_out = prenorm
            pn = (None if x_add is None else x_add.reshape(M, K), nw, eps,
                  None if x_out is None else x_out.view(M, K))
        Wd, sd = (wq, ws) if wq is not None else (w, None)
        y = ops.gemv(xm, Wd, sd, out=out, epilogue=epi, prenorm=pn, conv=conv)
        return residual if residual is not None else y.view(*x.shape[:-1], N)
    if conv is not None:
        raise ValueError("linear: the conv epilogue is a decode GEMV form (at most 8 fp32 rows, K a multiple of 256)")
    if prenorm is not None:
        x = prenorm_torch(x, prenorm)
    if wq is not None and K % 64 == 0 and x.dtype in (torch.float32, torch.int32, torch.bfloat16):
        y = ops.gemm_q8(x.reshape(M, K), wq, ws, out=out, epilogue="add" if epi == "add_fixed" else epi)
        return residual if residual is not None else y.view(*x.shape[:-1], N)
    if x.dtype == torch.int32:
        raise ValueError("linear: split activations need the int8 GEMM (int8 weights, K a multiple of 64)")
    if residual is not None:
        residual.view(M, N).addmm_(x.reshape(M, K), w.T)
        return residual
    return x @ w.T


def _fused(p, names):
    """The weights `names` of p stacked into one [sum N, H] weight (cached in p under "_in_fused"), with the stacked
    int8 rows and scales under "_in_fused.q" / "_in_fused.s" when every one has an int8 form."""
    w = p.get("_in_fused")
    if w is None:
        w = torch.cat([p[n] for n in names], dim=0).contiguous()
        p["_in_fused"] = w
        if all(n + ".q" in p for n in names):
            p["_in_fused.q"] = torch.cat([p[n + ".q"] for n in names], dim=0).contiguous()
            p["_in_fused.s"] = torch.cat([p[n + ".s"] for n in names], dim=0).contiguous()
    return w


def _q8(p, name):
    return p.get(name + ".q"), p.get(name + ".s")


def gdn_in_weight(p):
    """The four input projections of a Gated DeltaNet layer stacked into one [C + Vd + 2 Hv, H] weight (cached in p
    under "_in_fused")."""
    return _fused(p, ("in_proj_qkv", "in_proj_z", "in_proj_b", "in_proj_a"))


def attn_in_weight(p):
    """q_proj, k_proj and v_proj stacked into one [Hq 2D + 2 Hkv D, H] weight (cached in p under "_in_fused")."""
    return _fused(p, ("q_proj", "k_proj", "v_proj"))


def gated_attention_layer(x, p, k_cache, v_cache, pos, *, rope_theta=1e7, partial_rotary_factor=0.25, eps=1e-6,
                          cache_len=None, prenorm=None, residual=None, fixed_order=False):
    """Gated softmax attention mixer of one decoder layer (Qwen3_5Attention.forward, HF:656-701; WGSL attnPrep +
    attention, engine/kernels_qwen35.js:18-123). x: [B, T, H] fp32; the T tokens sit at positions pos..pos+T-1,
    pos a Python int or a [B] int32 device tensor (per row; a device tensor keeps the call capturable in a HIP
    graph). Their rotated keys and values are written into the caches at those positions, and token t attends to
    cache positions 0..pos+t (engine/kernels_qwen35.js:90). T > 1 at the int position 0 runs the flash prefill over
    the call's own tokens (for an fp32 y with the front end in its pre-pass, q35_gated_attn_prefill_proj); T > 1 at
    any other position (or a device pos) the same kernel over the cache (the caches' max_len must then be a multiple
    of 64; for an fp32 y with the front end in its pre-pass, q35_gated_attn_prefill_cached_proj); T == 1 the split-K
    decode over cache positions 0..pos (cache_len: optional [B] int32 per-row lengths, default pos + 1; without it
    the q / k norms, RoPE and the cache append run inside the decode kernels, q35_gated_attn_decode_proj, instead of
    a front-end launch). prenorm: see linear(). For T > 1, x may be the int32 words of split activations (see
    gated_deltanet_layer). Returns y [B, T, H], or with residual [B, T, H] given,
    residual + y computed in place by o_proj (then returned). fixed_order: see linear()."""
    B, T, _ = x.shape
    D = p["q_norm"].numel()
    Hq = p["q_proj"].shape[0] // (2 * D)
    Hkv = p["k_proj"].shape[0] // D
    rot = int(D * partial_rotary_factor)
    max_len = k_cache.shape[2]
    if torch.is_tensor(pos):
        pos_t = pos
        own_keys = False
    else:
        if pos < 0 or pos + T > max_len:
            raise ValueError(f"gated_attention_layer: positions {pos}..{pos + T - 1} exceed the cache ({max_len})")
        pos_t = torch.full((B,), int(pos), dtype=torch.int32, device=x.device)
        own_keys = pos == 0
    cos, sin = rope_tables(max_len, rot, rope_theta, x.device)
    y = linear(x, attn_in_weight(p), *_q8(p, "_in_fused"), prenorm=prenorm)
    if T == 1 and cache_len is None and y.dtype == torch.float32 and y.shape[-1] % 4 == 0:
        # one token: the front end (q / k norms, RoPE, cache append) runs inside the decode kernels, reading y
        o = ops.gated_attention_decode_proj(y, p["q_norm"], p["k_norm"], k_cache, v_cache, pos_t, cos, sin,
                                            num_heads=Hq, eps=eps, scale=1.0 / math.sqrt(D),
                                            out_dtype=torch.float32).view(B, 1, Hq * D)
        wq_o, ws_o = _q8(p, "o_proj")
        return linear(o, p["o_proj"], wq_o, ws_o, residual=residual, fixed_order=fixed_order)
    if T > 1 and own_keys and y.dtype == torch.float32 and y.shape[-1] % 4 == 0:
        # the call's own tokens: the front end runs in the prefill's pre-pass, reading y (q35_gated_attn_prefill_proj)
        o = ops.gated_attention_prefill_proj(y, p["q_norm"], p["k_norm"], k_cache, v_cache, cos, sin, num_heads=Hq,
                                             pos0=0, eps=eps, scale=1.0 / math.sqrt(D))
        wq_o, ws_o = _q8(p, "o_proj")
        xo = o if (wq_o is not None and o.shape[-1] % 64 == 0) else o.float()
        return linear(xo, p["o_proj"], wq_o, ws_o, residual=residual, fixed_order=fixed_order)
    if T > 1 and not own_keys and y.dtype == torch.float32 and y.shape[-1] % 4 == 0 and max_len % 64 == 0:
        # the same over the cache (tokens at per-row positions), the front end in the pre-pass
        # (q35_gated_attn_prefill_cached_proj)
        o = ops.gated_attention_prefill_cached_proj(y, p["q_norm"], p["k_norm"], k_cache, v_cache, pos_t, cos, sin,
                                                    num_heads=Hq, eps=eps, scale=1.0 / math.sqrt(D))
        wq_o, ws_o = _q8(p, "o_proj")
        xo = o if (wq_o is not None and o.shape[-1] % 64 == 0) else o.float()
        return linear(xo, p["o_proj"], wq_o, ws_o, residual=residual, fixed_order=fixed_order)
    q, gate, k, v = ops.attn_prep(y, p["q_norm"], p["k_norm"], cos, sin, pos_t, k_cache, v_cache, num_heads=Hq,
                                  num_kv_heads=Hkv, eps=eps, want_kv=T > 1 and own_keys)
    if T > 1 and own_keys:
        o = ops.gated_attention_prefill(q, k, v, gate, cos, sin, pos0=0, scale=1.0 / math.sqrt(D))
    elif T > 1:
        o = ops.gated_attention_prefill_cached(q, k_cache, v_cache, gate, pos_t, cos, sin, scale=1.0 / math.sqrt(D))
    else:
        cl = pos_t + 1 if cache_len is None else cache_len
        # fp32 straight from the merge kernel: the o_proj GEMV reads fp32 (no conversion kernel in the step)
        o = ops.gated_attention_decode(q[:, 0], k_cache, v_cache, gate[:, 0], cl, cos, sin,
                                       scale=1.0 / math.sqrt(D), out_dtype=torch.float32).view(B, 1, Hq * D)
    wq_o, ws_o = _q8(p, "o_proj")
    # bf16 o straight into the int8 GEMM (the product of o.float(), bitwise); fp32 for the other forms
    xo = o if (T > 1 and wq_o is not None and o.shape[-1] % 64 == 0) else o.float()
    return linear(xo, p["o_proj"], wq_o, ws_o, residual=residual, fixed_order=fixed_order)


def residual_steer_add(x, vecs, rows=None):
    """x[r, t, :] += vecs[rows[r]] at every position t, in place (the layers[l] forward hook of
    tests/engine_ref.py:49-53 and the WGSL resAdd of engine/kernels.js:190-203). rows: [B] int, -1 for no vector;
    None gives row r the vector min(r, nvec - 1) as the WGSL's clamped row index does. Returns x."""
    if rows is not None and not torch.is_tensor(rows):
        rows = torch.as_tensor(rows, dtype=torch.int32, device=x.device)
    return ops.residual_steer_add_(x, vecs, rows)
