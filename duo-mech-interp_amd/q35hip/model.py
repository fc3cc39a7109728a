"""Qwen3.5-shaped hybrid decoder stack on one MI355X: the hot path runs on the q35hip HIP ops, the glue around it
(projections, causal conv, norms, int8-dequantised SwiGLU, embedding, lm head) on torch.

The layer loop follows Model._forward (engine/model.js:404-466) and Qwen3_5DecoderLayer.forward (HF: transformers
5.15.0 models/qwen3_5/modeling_qwen3_5.py, HF:753-793): RMSNorm(1 + w) -> mixer -> + residual -> RMSNorm(1 + w) ->
SwiGLU MLP -> + residual -> [steering add]. The mixers and the steering add are the per-layer functions of
q35hip.layers; the model owns their states (GDN conv / recurrent states, bf16 KV caches) and mutates them in place
(engine/model.js:308-342).
"""
import torch

from . import layers, ops
from .workloads import dequantize_int8


class Q35Weights:
    """Device copy of a weight dict: fp32 tensors as given; each int8 weight (keys "<name>.q" int8 [N, K] and
    "<name>.s" fp32 [N, K / 128] per group of 128 inputs, or [N] per row) both kept as int8 + scales (for the GEMVs
    and GEMMs) and dequantised once to fp32 under "<name>" (for the embedding lookup and torch fallbacks of shapes the
    kernels do not take)."""

    def __init__(self, W, device):
        self.t = {}
        for k, v in W.items():
            if k.endswith(".q"):
                base = k[:-2]
                self.t[base] = dequantize_int8(v, W[base + ".s"]).to(device)
                self.t[k] = v.to(device).contiguous()
            elif k + ".q" not in W:  # a dequantised copy given beside its int8 form is rebuilt from the int8 above
                self.t[k] = v.to(device)

    def __getitem__(self, k):
        return self.t[k]


MAX_PUSHES = 8  # neuron pushes per layer (engine/model.js:415)
_NO_PUSH = (1 << 30, 0, 0, 0, 0, 0)  # a record that matches no neuron (neuron index past any layer width)


def mlp_weights(p):
    """Per-layer MLP buffers (cached in p): "_gu" the [gate | up] fp32 weight (the torch path without int8 weights),
    "_gu_q8" / "_gu_s" the int8 rows interleaved (gate j, up j) for the SwiGLU epilogues of the decode GEMV and the
    prefill GEMM, "_pushes" the layer's push records."""
    if "_gu" not in p:
        p["_gu"] = torch.cat([p["gate_proj"], p["up_proj"]], dim=0).contiguous()
        if "gate_proj.q" in p:
            I, H = p["gate_proj.q"].shape
            p["_gu_q8"] = torch.stack([p["gate_proj.q"], p["up_proj.q"]], dim=1).reshape(2 * I, H).contiguous()
            gs = p["gate_proj.s"]
            p["_gu_s"] = torch.stack([gs, p["up_proj.s"]], dim=1).reshape(2 * I, *gs.shape[1:]).contiguous()
        p["_pushes"] = torch.tensor([_NO_PUSH] * MAX_PUSHES, dtype=torch.int32, device=p["_gu"].device)
    return p


_GDN_IN = ("in_proj_qkv", "in_proj_z", "in_proj_b", "in_proj_a")
_ATTN_IN = ("q_proj", "k_proj", "v_proj")
_MLP_IN = ("gate_proj", "up_proj")


def _split_ok(p, names, x):
    """Whether the products that read a norm's output all run on the int8 GEMM (int8 weights, 64 | H), which then
    takes the rows already split."""
    return x.shape[-1] % 64 == 0 and all(n + ".q" in p for n in names)


def mlp(p, h, x, prenorm=None, capture=None, fixed_order=False):
    """x += SwiGLU MLP (HF:704-717) of h, in place, with the layer's neuron pushes at the down_proj input
    (engine/model.js:7-9, engine/kernels_qwen35.js:250-279). Decode (at most 8 rows, int8 weights present): one GEMV
    over the interleaved int8 gate/up rows with the SwiGLU + push epilogue, and one int8 GEMV accumulating down_proj
    into x. Prefill (more rows): the int8 GEMM with the same SwiGLU + push epilogue over the interleaved rows, then an
    int8 GEMM accumulating down_proj into x; without int8 weights a [gate | up] torch GEMM on the fp32 weights, the
    SwiGLU push kernel and a down_proj GEMM. prenorm = (y_add, norm_w, eps): h is then the residual; x receives
    h + y_add and the MLP reads the RMSNorm (1 + norm_w) of that sum (the layer's second add + norm, fused into the
    first GEMV on the decode path). h may be the int32 words of split activations (add_rmsnorm_(..., split=True)) when
    the layer has int8 weights: the gate/up GEMM reads them as they are. capture: an fp32 view [rows, T, I] (unit
    neuron stride) that receives the post-push activations, the down_proj input (the engine's capture hook,
    engine/model.js:9, :451-453), written by the SwiGLU epilogue itself. fixed_order: the decode down_proj sums
    every output in one fixed order (repeatable bits; layers.linear). Returns x."""
    mlp_weights(p)
    H = h.shape[-1]
    M = h.numel() // H
    T = h.shape[1] if h.dim() == 3 else 1
    # h + y_add is written to x when x is another buffer; with x = h and no y_add the norm reads h as it is
    pn = None if prenorm is None else (prenorm[0], prenorm[1], prenorm[2], None if x is h else x)
    if M <= 8 and "_gu_q8" in p and H % 256 == 0 and p["down_proj.q"].shape[1] % 256 == 0 and \
            h.dtype == torch.float32:
        pn2 = None if pn is None else (None if pn[0] is None else pn[0].reshape(M, H), pn[1], pn[2],
                                       None if pn[3] is None else x.view(M, H))
        a = ops.gemv(h.reshape(M, H), p["_gu_q8"], p["_gu_s"], epilogue="swiglu", pushes=p["_pushes"], T=T,
                     prenorm=pn2, capture=capture)
        ops.gemv(a, p["down_proj.q"], p["down_proj.s"], out=x.view(M, H),
                 epilogue="add_fixed" if fixed_order else "add")
        return x
    if pn is not None:
        h = layers.prenorm_torch(h, pn)
    if "_gu_q8" in p and H % 64 == 0 and p["down_proj.q"].shape[1] % 64 == 0:
        # int8 GEMMs: [gate | up] interleaved with the SwiGLU + push epilogue (its output already split for the next
        # product), then down_proj accumulating into x
        a = ops.gemm_q8(h.reshape(M, H), p["_gu_q8"], p["_gu_s"], epilogue="swiglu", pushes=p["_pushes"], T=T,
                        split_out=p["_gu_q8"].shape[0] % 16 == 0, capture=capture)
        ops.gemm_q8(a, p["down_proj.q"], p["down_proj.s"], out=x.view(M, H), epilogue="add")
        return x
    if h.dtype == torch.int32:
        raise ValueError("mlp: split activations need the int8 GEMM (int8 weights, H a multiple of 64)")
    a = ops.swiglu_push(h @ p["_gu"].T, p["_pushes"], T=T, capture=capture)
    x.view(M, H).addmm_(a.view(M, -1), p["down_proj"].T)
    return x


class HybridModel:
    """B independent rows decoded together (the boosted / as-is / suppressed rows of the reference's steer loop,
    engine/analysis.js:117-145). fp32 residual stream; vectors added after steer_layer at every position.

    gdn_prefill selects the Gated DeltaNet prefill kernel: "chunk" (default) runs the chunked form, which on the
    stack's fp32 activations computes every product in fp32 (agreement with the fp32 CPU recurrence to about 1e-6,
    so greedy tokens follow the fp32 reference through near ties of a few 1e-3 in the logits); "recurrent" runs the
    token-serial fp32 kernel (the WGSL engine's order, token by token; slower).

    Each row has its own position (rows may hold prompts of different lengths, prefilled one row at a time as the
    reference's steer loop does: reset(r); forward(ids_r, row=r), engine/analysis.js:125), and a prompt may be
    prefilled in several calls (engine/model.js:486-491): a multi-token call past position 0 attends over the KV
    cache. Positions live on the device (pos_dev, [rows] int32) and the steering vectors in fixed buffers, so a
    decode step has no host-dependent arguments: enable_decode_graph() captures one step in a HIP graph that
    decode_step() replays.

    deterministic: the decode step's residual adds (the mixers' output projections and down_proj) sum every output
    in one fixed order, so that two runs give identical logits bit for bit; by default these N = hidden products
    split K over four blocks that add with fp32 atomics (faster; the last bits of a step may vary between runs).
    Prefill is deterministic either way."""

    MAX_VECS = 4  # vector rows of the steering buffer (the WGSL resAdd clamps its row index to 3, engine/kernels.js:201)

    def __init__(self, cfg, W, device, max_len=4096, rows=3, steer_layer=12, gdn_prefill="chunk",
                 deterministic=False):
        if gdn_prefill not in ("chunk", "recurrent"):
            raise ValueError(f"HybridModel: gdn_prefill must be 'chunk' or 'recurrent', not {gdn_prefill!r}")
        self.cfg, self.device, self.steer_layer = cfg, device, steer_layer
        self.gdn_prefill = gdn_prefill
        self.deterministic = bool(deterministic)
        self.W = W if isinstance(W, Q35Weights) else Q35Weights(W, device)
        # the KV caches hold a multiple of 64 positions (the multi-token attention over the cache reads 64-key tiles)
        self.max_len, self.rows = (max_len + 63) // 64 * 64, rows
        self.vec_buf = torch.zeros(self.MAX_VECS, cfg.hidden, device=device)
        self.vec_rows = torch.full((rows,), -1, dtype=torch.int32, device=device)
        self.steering = False
        self.params = [{n[len(f"layers.{l}."):]: t for n, t in self.W.t.items() if n.startswith(f"layers.{l}.")}
                       for l in range(cfg.layers)]
        for l, p in enumerate(self.params):  # stacked input projections and MLP buffers, built once
            if cfg.is_attention(l):
                layers.attn_in_weight(p)
            else:
                layers.gdn_in_weight(p)
                # the engine's per-head output scale (engine/model.js:362-368): 1 for every head until set
                p["_head_scale"] = torch.ones(cfg.lin_v_heads, device=device)
            mlp_weights(p)
        self.states = []
        for l in range(cfg.layers):
            if cfg.is_attention(l):
                shape = (rows, cfg.n_kv, self.max_len, cfg.head_dim)
                self.states.append({"k": torch.zeros(shape, dtype=torch.bfloat16, device=device),
                                    "v": torch.zeros(shape, dtype=torch.bfloat16, device=device)})
            else:
                self.states.append({
                    "conv": torch.zeros(rows, cfg.conv_k - 1, cfg.conv_dim, device=device),
                    "rec": torch.zeros(rows, cfg.lin_v_heads, cfg.lin_dk, cfg.lin_dv, device=device)})
        # each row's next position, on the device (the decode step reads it there, so a replayed graph follows it)
        self.pos_dev = torch.zeros(rows, dtype=torch.int32, device=device)
        # the LM head's argmax slots (q35_gemv_norm_argmax: zeros between calls)
        self._amax_slots = torch.zeros(rows, dtype=torch.int64, device=device)
        self.graph = None
        self.step_capture, self._step_cap_idx = None, {}
        self.row_pos = [0] * rows  # host mirror of pos_dev
        self.reset()

    def reset(self, row=None):
        """Start a new sequence on every row, or on row `row` only: zero its recurrent and conv states and its
        position (KV caches are overwritten by position)."""
        rs = slice(None) if row is None else slice(row, row + 1)
        for st in self.states:
            if "rec" in st:
                st["rec"][rs].zero_()
                st["conv"][rs].zero_()
        self.pos_dev[rs].zero_()
        for r in range(self.rows)[rs]:
            self.row_pos[r] = 0

    @property
    def pos(self):
        """The furthest row's next position (all rows share it unless rows were prefilled separately)."""
        return max(self.row_pos)

    def set_vectors(self, vecs, vec_of_row):
        """vecs: [n, H] fp32 (n <= MAX_VECS), copied into the model's buffer; vec_of_row: [rows] int (-1 = no vector).
        None clears the steering."""
        if vecs is None:
            self.vec_rows.fill_(-1)
            self.steering = False
            return
        vecs = vecs.to(self.device, torch.float32)
        if vecs.shape[0] > self.MAX_VECS:
            raise ValueError(f"HybridModel: at most {self.MAX_VECS} steering vectors")
        self.vec_buf[:vecs.shape[0]].copy_(vecs)
        self.vec_rows.copy_(torch.as_tensor(vec_of_row, dtype=torch.int32))
        self.steering = True

    def set_head_scales(self, scales):
        """Per-head output scales of the Gated DeltaNet layers, {layer: [Hv] values} (the engine's `heads` ablation
        hook, engine/model.js:10, :362-368): applied after the gated norm (engine/kernels_qwen35.js:243); heads of
        layers not named (or scales None) get 1. Written into fixed per-layer buffers, so a captured decode step picks
        them up."""
        for l, p in enumerate(self.params):
            if "_head_scale" not in p:
                if scales and l in scales:
                    raise ValueError(f"HybridModel: layer {l} is not a Gated DeltaNet layer")
                continue
            s = scales.get(l) if scales else None
            if s is None:
                p["_head_scale"].fill_(1.0)
            else:
                s = torch.as_tensor(s, dtype=torch.float32).reshape(-1)
                if s.numel() != p["_head_scale"].numel():
                    raise ValueError(f"HybridModel: layer {l} takes {p['_head_scale'].numel()} head scales")
                p["_head_scale"].copy_(s)

    def set_pushes(self, pushes):
        """Neuron pushes per layer, {layer: [(neuron or None for every neuron, "add" | "mul", [value per row])]}, at
        most 8 per layer (engine/model.js:412-423); layers not named have none. Written into fixed per-layer buffers,
        so a captured decode step picks them up."""
        for l, p in enumerate(self.params):
            recs = pushes.get(l, []) if pushes else []
            if len(recs) > MAX_PUSHES:
                raise ValueError(f"HybridModel: at most {MAX_PUSHES} pushes per layer")
            buf = torch.tensor([_NO_PUSH] * MAX_PUSHES, dtype=torch.int32)
            if recs:
                buf[:len(recs)] = ops.pack_pushes(recs, "cpu")
            p["_pushes"].copy_(buf)

    def _layers(self, x, T, last, collect_layer, steer, rs=slice(None), attn_pos=None, hooks=None):
        """The decoder layers 0..last over the residual stream x [n, T, H] (dense fp32) of the rows rs; returns (the
        residual after layer `last`, the residual after collect_layer or None) (HF:753-793; engine/model.js:436-462).
        attn_pos: the attention layers' position argument for T > 1 (0 when every row starts its sequence: the
        prefill over the call's own keys; else the rows' device positions: the prefill over the KV cache).

        Prefill (T > 1): x is updated in place; each layer adds its mixer output in the fused residual-add + RMSNorm
        kernel and its MLP output in the MLP's last product. Decode (T == 1): x is updated in place by the GEMVs:
        the mixer's input projection and the MLP's first GEMV normalise the residual in their prologue
        (q35_gemv_norm), and the mixer's output projection and down_proj accumulate into it (split over K, so that
        these N = hidden products draw bandwidth from every CU).

        hooks (the engine's forward options, engine/model.js:9-11, :446-461): "cap" = (buffer [nL, n, capT, I],
        {layer: index}, t0): the MLP activations of the listed layers written by the SwiGLU epilogues at tokens
        t0 .. t0 + T - 1; "resid" = (buffer [last + 1, n, capT, H], mode, t0): the residual after every layer
        (mode "layer", after the steering add) or after the mixer's residual add (mode "mixer", the engine's
        resid "attn")."""
        cfg = self.cfg
        collected = None
        hooks = hooks or {}
        cap_buf, cap_idx, cap_t0 = hooks.get("cap", (None, {}, 0))
        res_buf, res_mode, res_t0 = hooks.get("resid", (None, "layer", 0))

        def cap_view(l):
            i = cap_idx.get(l)
            return None if i is None else cap_buf[i, :, cap_t0:cap_t0 + T]

        def snap(l, mode):
            if res_buf is not None and res_mode == mode:
                res_buf[l, :, res_t0:res_t0 + T].copy_(x.view(res_buf.shape[1], T, -1))
        pos_dev, vec_rows = self.pos_dev[rs], self.vec_rows[rs]
        if T == 1:
            fx = self.deterministic
            for l in range(last + 1):
                p = self.params[l]
                st = {n: t[rs] for n, t in self.states[l].items()}
                pre = (None, p["input_layernorm"], cfg.eps, None)
                if cfg.is_attention(l):
                    layers.gated_attention_layer(x, p, st["k"], st["v"], pos_dev, rope_theta=cfg.rope_theta,
                                                 partial_rotary_factor=cfg.partial_rotary, eps=cfg.eps,
                                                 prenorm=pre, residual=x, fixed_order=fx)
                else:
                    layers.gated_deltanet_layer(x, p, st["conv"], st["rec"], p["_head_scale"],
                                                num_k_heads=cfg.lin_k_heads, head_k_dim=cfg.lin_dk, eps=cfg.eps,
                                                prefill=self.gdn_prefill, prenorm=pre, residual=x, fixed_order=fx)
                snap(l, "mixer")
                mlp(p, x, x, prenorm=(None, p["post_attention_layernorm"], cfg.eps), capture=cap_view(l),
                    fixed_order=fx)
                if l == self.steer_layer and steer:
                    layers.residual_steer_add(x, self.vec_buf, vec_rows)
                snap(l, "layer")
                if l == collect_layer:
                    collected = x.clone()
            return x, collected
        y = None  # the previous mixer's output, added to x by the next norm
        for l in range(last + 1):
            p = self.params[l]
            st = {n: t[rs] for n, t in self.states[l].items()}
            # the norms hand the int8 GEMMs their rows already split (bf16 hi + lo) when the layer's products are int8
            mixer = _ATTN_IN if cfg.is_attention(l) else _GDN_IN
            h = ops.add_rmsnorm_(x, y, p["input_layernorm"], cfg.eps, split=_split_ok(p, mixer, x))
            if cfg.is_attention(l):
                y = layers.gated_attention_layer(h, p, st["k"], st["v"], attn_pos, rope_theta=cfg.rope_theta,
                                                 partial_rotary_factor=cfg.partial_rotary, eps=cfg.eps)
            else:
                y = layers.gated_deltanet_layer(h, p, st["conv"], st["rec"], p["_head_scale"],
                                                num_k_heads=cfg.lin_k_heads, head_k_dim=cfg.lin_dk, eps=cfg.eps,
                                                prefill=self.gdn_prefill)
            h = ops.add_rmsnorm_(x, y, p["post_attention_layernorm"], cfg.eps, split=_split_ok(p, _MLP_IN, x))
            y = None
            snap(l, "mixer")
            mlp(p, h, x, capture=cap_view(l))
            if l == self.steer_layer and steer:
                layers.residual_steer_add(x, self.vec_buf, vec_rows)
            snap(l, "layer")
            if l == collect_layer:
                collected = x.clone()
        return x, collected

    @torch.no_grad()
    def forward(self, ids, stop_after=None, collect_layer=None, row=None, *, capture=None, capture_layers=None,
                resid=None, resid_mode="layer", t0=0):
        """ids: [rows, T] token ids continuing every row's sequence, or with row=r [1, T] (or [T]) continuing row r
        only (its states and position; the other rows are untouched). A multi-token call may start anywhere: past
        position 0 its attention runs over the KV cache. Returns (last-position logits [n, V] or None with
        stop_after, residual after collect_layer or None) for the rows called.

        The engine's forward hooks (engine/model.js:9-11, :446-461; device buffers owned by the caller, n = rows
        called, capT >= t0 + T, so a prompt given in several calls fills one buffer through t0, as the engine's capT0):
          capture  fp32 [len(capture_layers), n, capT, I]: the MLP activations (the down_proj input, after the
                   pushes) of every token, written by the SwiGLU epilogues; capture_layers defaults to every layer
          resid    fp32 [layers run, n, capT, H]: the residual stream after each layer (resid_mode "layer", after
                   the steering add) or after each mixer's residual add (resid_mode "mixer", the engine's "attn")"""
        cfg, W = self.cfg, self.W
        if row is None:
            rs, rows = slice(None), list(range(self.rows))
        else:
            if not 0 <= row < self.rows:
                raise ValueError(f"HybridModel: row {row} out of range ({self.rows} rows)")
            rs, rows = slice(row, row + 1), [row]
            ids = ids.reshape(1, -1)
        T = ids.shape[1]
        if max(self.row_pos[r] for r in rows) + T > self.max_len:
            raise ValueError("context exceeds the KV cache")
        attn_pos = 0 if all(self.row_pos[r] == 0 for r in rows) else self.pos_dev[rs]
        x = W["embed"][ids.to(self.device).long()].contiguous()
        last = cfg.layers - 1 if stop_after is None else stop_after
        hooks = self._hooks(len(rows), T, last, capture, capture_layers, resid, resid_mode, t0)
        x, collected = self._layers(x, T, last, collect_layer, self.steering, rs, attn_pos, hooks)
        self.pos_dev[rs].add_(T)
        for r in rows:
            self.row_pos[r] += T
        if stop_after is not None:
            return None, collected
        return self._lm_head(x[:, -1]), collected

    def _hooks(self, n, T, last, capture, capture_layers, resid, resid_mode, t0):
        """Validated hook buffers of a forward call (see forward)."""
        cfg, hooks = self.cfg, {}
        if capture is not None:
            lays = list(range(cfg.layers)) if capture_layers is None else [int(l) for l in capture_layers]
            if any(not 0 <= l < cfg.layers for l in lays) or len(set(lays)) != len(lays):
                raise ValueError("HybridModel: capture_layers must be distinct layer indices")
            if (capture.dtype != torch.float32 or capture.device != self.device or capture.dim() != 4
                    or tuple(capture.shape[:2]) != (len(lays), n) or capture.shape[3] != cfg.inter
                    or not 0 <= t0 <= capture.shape[2] - T or capture.stride(3) != 1):
                raise ValueError(f"HybridModel: capture must be fp32 [{len(lays)}, {n}, >= t0 + {T}, {cfg.inter}] "
                                 "on the model's device")
            hooks["cap"] = (capture, {l: i for i, l in enumerate(lays)}, int(t0))
        if resid is not None:
            if resid_mode not in ("layer", "mixer"):
                raise ValueError(f"HybridModel: resid_mode must be 'layer' or 'mixer', not {resid_mode!r}")
            if (resid.dtype != torch.float32 or resid.device != self.device or resid.dim() != 4
                    or resid.shape[0] < last + 1 or resid.shape[1] != n or resid.shape[3] != cfg.hidden
                    or not 0 <= t0 <= resid.shape[2] - T):
                raise ValueError(f"HybridModel: resid must be fp32 [>= {last + 1}, {n}, >= t0 + {T}, {cfg.hidden}] "
                                 "on the model's device")
            hooks["resid"] = (resid, resid_mode, int(t0))
        return hooks

    def _lm_head(self, xl, ids_out=None):
        """Final RMSNorm and the tied-embedding logits of the last positions xl [rows, H] (a GEMV for few rows).
        ids_out: also each row's greedy pick (argmax of the logits) into this [rows] int32 buffer, folded into the
        LM head's GEMV when its weights are int8 (q35_gemv_norm_argmax), else ops.argmax_rows."""
        head = "lm_head" if "lm_head" in self.W.t else "embed"  # untied checkpoints carry their own head
        wq = self.W.t.get(head + ".q")
        xl = xl.contiguous()
        pre = (None, self.W["norm"], self.cfg.eps, None)
        if (ids_out is not None and wq is not None and xl.shape[0] <= 8 and xl.shape[-1] % 256 == 0
                and xl.dtype == torch.float32):
            return ops.gemv_norm_argmax(xl, wq, self.W[head + ".s"], pre, self._amax_slots, idx=ids_out)[0]
        logits = layers.linear(xl, self.W[head], wq, None if wq is None else self.W[head + ".s"], prenorm=pre)
        if ids_out is not None:
            ops.argmax_rows(logits, out=ids_out)
        return logits

    def set_step_capture(self, capture_layers):
        """Capture the MLP activations of `capture_layers` (None: stop) at every decode step (decode_step,
        decode_greedy, graph or eager) into self.step_capture [len(layers), rows, 1, I] fp32, overwritten by each step.
        Call before enable_decode_graph(): the graph records the buffer it finds."""
        if capture_layers is None:
            self.step_capture, self._step_cap_idx = None, {}
            return
        lays = [int(l) for l in capture_layers]
        if any(not 0 <= l < self.cfg.layers for l in lays) or len(set(lays)) != len(lays):
            raise ValueError("HybridModel: capture_layers must be distinct layer indices")
        self.step_capture = torch.zeros(len(lays), self.rows, 1, self.cfg.inter, device=self.device)
        self._step_cap_idx = {l: i for i, l in enumerate(lays)}

    def _step_hooks(self):
        cap = self.step_capture
        return {} if cap is None else {"cap": (cap, self._step_cap_idx, 0)}

    @torch.no_grad()
    def enable_decode_graph(self):
        """Capture one decode step in a HIP graph: ids [rows] int32 (self._g_ids) -> logits, then the device argmax of
        the logits written back into self._g_ids, so that replaying the graph again continues greedy decoding with no
        host work (the engine's decode loop, engine/model.js:494-497). decode_step() and decode_greedy() replay it.
        Must be called at the start of a sequence: the warm-up runs real steps, and the states are reset afterwards.
        The steering add is always part of the graph (rows without a vector are skipped by the kernel), and so are the
        neuron pushes, the head scales and the step capture (set_step_capture) in their fixed buffers."""
        cfg = self.cfg
        self.reset()
        self._g_ids = torch.zeros(self.rows, dtype=torch.int32, device=self.device)
        hooks = self._step_hooks()

        def step():
            x, _ = self._layers(self.W["embed"].index_select(0, self._g_ids).unsqueeze(1), 1, cfg.layers - 1, None,
                                True, hooks=hooks)
            self.pos_dev.add_(1)
            return self._lm_head(x[:, -1], ids_out=self._g_ids)
        side = torch.cuda.Stream(device=self.device)
        side.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(side):  # warm-up outside capture: library handles, allocator pools
            for _ in range(2):
                step()
        torch.cuda.current_stream(self.device).wait_stream(side)
        torch.cuda.synchronize(self.device)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            self._g_logits = step()
        self.graph = g
        torch.cuda.synchronize(self.device)
        self.reset()
        self._g_ids.zero_()

    @torch.no_grad()
    def decode_step(self, ids):
        """One step for every row: ids [rows] or [rows, 1]. Replays the captured graph when there is one (the returned
        logits then live in the graph's output buffer, overwritten by the next step), else runs forward."""
        ids = ids.reshape(self.rows)
        if self.graph is None:
            cap = self.step_capture
            lays = None if cap is None else sorted(self._step_cap_idx, key=self._step_cap_idx.get)
            return self.forward(ids.reshape(self.rows, 1), capture=cap, capture_layers=lays)[0]
        if self.pos + 1 > self.max_len:
            raise ValueError("context exceeds the KV cache")
        self._g_ids.copy_(ids)
        self.graph.replay()
        self.row_pos = [p + 1 for p in self.row_pos]
        return self._g_logits

    @torch.no_grad()
    def decode_greedy(self):
        """One greedy step continuing from the last one (graph mode): replays the graph on the token ids the previous
        step's device argmax left in self._g_ids. Returns (logits, next ids [rows] int32), both graph buffers."""
        if self.graph is None:
            raise ValueError("decode_greedy needs enable_decode_graph()")
        if self.pos + 1 > self.max_len:
            raise ValueError("context exceeds the KV cache")
        self.graph.replay()
        self.row_pos = [p + 1 for p in self.row_pos]
        return self._g_logits, self._g_ids


@torch.no_grad()
def greedy(model, prompt_ids, steps):
    """Prefill prompt_ids [B, T], then `steps` greedy tokens (the device argmax: lowest index on ties, as torch.argmax
    and the WGSL argmax of engine/kernels.js:260-283). Returns (tokens [B, steps], top-2 margins [B, steps]) on the
    CPU."""
    logits, _ = model.forward(prompt_ids)
    toks, margins = [], []
    for _ in range(steps):
        top2 = logits.topk(2, dim=-1)
        nxt = ops.argmax_rows(logits)
        toks.append(nxt.long())
        margins.append(top2.values[:, 0] - top2.values[:, 1])
        logits = model.decode_step(nxt)
    return torch.stack(toks, 1).cpu(), torch.stack(margins, 1).cpu()


def median_resid_norm(resid_row):
    """Median over tokens 1..T-1 of |x_t| (engine/analysis.js:64-74: sorted, element len >> 1)."""
    n = resid_row[1:].float().norm(dim=-1).sort().values
    return float(n[n.shape[0] >> 1])


@torch.no_grad()
def steered_greedy(model, prompt_ids, steps, steer_layer=12, dose=0.8, seed=0):
    """The three-row steering protocol: a randn(H) vector (seed `seed`) scaled to `dose` x the median residual norm
    after `steer_layer` of the unsteered prompt (tokens 1..T-1), added on row 0, absent on row 1, negated on row 2,
    at every position of the prefill and of each greedy step (engine/analysis.js:117-145 with vec rows
    [+v, none, -v] as tests/engine.html:84 sets them). Returns (tokens, margins, vector)."""
    cfg = model.cfg
    model.reset()
    model.set_vectors(None, None)
    # the states are sized for every row, so the unsteered calibration pass runs the whole batch and reads row 0
    _, resid = model.forward(prompt_ids, stop_after=steer_layer, collect_layer=steer_layer)
    med = median_resid_norm(resid[0])
    v = torch.randn(cfg.hidden, generator=torch.Generator().manual_seed(seed))
    v = v / v.norm() * (dose * med)
    model.set_vectors(torch.stack([v, -v]), [0, -1, 1])
    model.reset()
    toks, margins = greedy(model, prompt_ids, steps)
    return toks, margins, v
