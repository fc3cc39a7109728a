"""Qwen3.5 checkpoints from a local directory: the HF layout the engine streams (config.json plus one or more
*.safetensors files, engine/model.js:21-23, :70-116, :153-280) turned into the weight dict of HybridModel.

Every linear layer and the embedding are quantized to int8 on load, as the engine does (engine/model.js:3-5), in the
engine's format: one fp32 scale per group of 128 inputs of a row (engine/kernels.js:15-47,
q35hip.workloads.quantize_groups_int8). A layer whose input width is not a multiple of 128 is refused, as the
engine's _allocQ refuses it (engine/model.js:118-120); group=0 quantizes per output row instead. The quantized dict
is cached on disk, like the engine's q8 cache in Cache Storage (engine/model.js:140, :280), so a second load reads
int8 directly.

Tensors are read with safetensors (no pickle). Names: the multimodal checkpoints keep the text decoder under
"model.language_model." (engine/model.js:22), text-only ones under "model."; HF's per-layer names follow HF:426-429
and HF:641-654.
"""
import hashlib
import json
import os

import torch
from safetensors import safe_open
from safetensors.torch import save_file

from .workloads import QG, Q35Config, dequantize_int8, quantize_int8

_PREFIXES = ("model.language_model.", "model.")
_CACHE_VERSION = "q35-q8-v2"


def config_from_hf(cfg):
    """Q35Config from a config.json dict (the text part of a multimodal config is under "text_config", HFcfg:82-115)."""
    c = cfg.get("text_config", cfg)
    rope = c.get("rope_parameters") or {}
    layer_types = c.get("layer_types")
    kw = dict(vocab=c["vocab_size"], hidden=c["hidden_size"], inter=c["intermediate_size"],
              layers=c["num_hidden_layers"], n_heads=c["num_attention_heads"], n_kv=c["num_key_value_heads"],
              head_dim=c.get("head_dim", 256), lin_k_heads=c["linear_num_key_heads"],
              lin_v_heads=c["linear_num_value_heads"], lin_dk=c["linear_key_head_dim"],
              lin_dv=c["linear_value_head_dim"], conv_k=c.get("linear_conv_kernel_dim", 4),
              rope_theta=float(rope.get("rope_theta", c.get("rope_theta", 1e7))),
              partial_rotary=float(rope.get("partial_rotary_factor", c.get("partial_rotary_factor", 0.25))),
              eps=float(c.get("rms_norm_eps", 1e-6)),
              tie_embeddings=bool(c.get("tie_word_embeddings", cfg.get("tie_word_embeddings", True))))
    if layer_types is not None:
        kw["layer_types"] = tuple(layer_types)
    elif "full_attention_interval" in c:
        kw["full_attention_interval"] = int(c["full_attention_interval"])
    return Q35Config(**kw)


def _shards(path):
    """(tensor name -> shard file) of a checkpoint directory: model.safetensors.index.json when present, else every
    *.safetensors file."""
    idx = os.path.join(path, "model.safetensors.index.json")
    if os.path.exists(idx):
        wm = json.load(open(idx))["weight_map"]
        return {k: os.path.join(path, f) for k, f in wm.items()}
    out = {}
    for f in sorted(os.listdir(path)):
        if f.endswith(".safetensors"):
            with safe_open(os.path.join(path, f), framework="pt") as sf:
                for k in sf.keys():
                    out[k] = os.path.join(path, f)
    if not out:
        raise FileNotFoundError(f"no *.safetensors in {path}")
    return out


def _layer_names(cfg, l):
    """(our key, HF name relative to the prefix, kind) of layer l's tensors; kind "q" = linear to quantize, "f" =
    fp32 as is, "conv" = the [C, 1, K] depthwise conv weight."""
    hp = f"layers.{l}."
    out = [("input_layernorm", "input_layernorm.weight", "f"),
           ("post_attention_layernorm", "post_attention_layernorm.weight", "f")]
    for n in ("gate_proj", "up_proj", "down_proj"):
        out.append((n, f"mlp.{n}.weight", "q"))
    if cfg.is_attention(l):
        for n in ("q_proj", "k_proj", "v_proj", "o_proj"):
            out.append((n, f"self_attn.{n}.weight", "q"))
        out += [("q_norm", "self_attn.q_norm.weight", "f"), ("k_norm", "self_attn.k_norm.weight", "f")]
    else:
        for n in ("in_proj_qkv", "in_proj_z", "in_proj_b", "in_proj_a", "out_proj"):
            out.append((n, f"linear_attn.{n}.weight", "q"))
        out += [("norm", "linear_attn.norm.weight", "f"), ("conv1d", "linear_attn.conv1d.weight", "conv"),
                ("dt_bias", "linear_attn.dt_bias", "f"), ("A_log", "linear_attn.A_log", "f")]
    return [(f"layers.{l}.{k}", hp + n, kind) for k, n, kind in out]


def _cache_key(path, shard_files, int8, group):
    h = hashlib.sha1(_CACHE_VERSION.encode())
    h.update(os.path.abspath(path).encode())
    h.update(b"int8" if int8 else b"fp32")
    h.update(f"group{group}".encode())
    for f in sorted(set(shard_files)):
        st = os.stat(f)
        h.update(f"{os.path.basename(f)}:{st.st_size}:{int(st.st_mtime)}".encode())
    return h.hexdigest()[:24]


def _expand(W):
    """Add the dequantised fp32 "<name>" beside every "<name>.q" except the MLP's (HybridModel's weight format, as
    q35hip.workloads.init_weights writes it)."""
    for k in [k for k in W if k.endswith(".q")]:
        base = k[:-2]
        if not any(base.endswith(n) for n in ("gate_proj", "up_proj", "down_proj")):
            W[base] = dequantize_int8(W[k], W[base + ".s"])
    return W


def load_checkpoint(path, *, int8=True, cache_dir=None, group=QG):
    """(Q35Config, weight dict) of the Qwen3.5 checkpoint in directory `path`. int8: every linear and the embedding
    int8 with fp32 scales per group of `group` inputs, or per row with group 0 ("<name>.q", "<name>.s", plus the
    dequantised "<name>" except for the MLP); otherwise fp32 throughout (the MLP still int8, the form the stack's MLP
    reads). cache_dir (default <path>/.q35cache; False for none) keeps the quantized tensors for the next load."""
    cfg = config_from_hf(json.load(open(os.path.join(path, "config.json"))))
    shards = _shards(path)
    if cache_dir is None:
        cache_dir = os.path.join(path, ".q35cache")
    cache_file = None
    if cache_dir:
        cache_file = os.path.join(cache_dir, _cache_key(path, shards.values(), int8, group) + ".safetensors")
        if os.path.exists(cache_file):
            W = {}
            with safe_open(cache_file, framework="pt") as sf:
                for k in sf.keys():
                    W[k] = sf.get_tensor(k)
            return cfg, _expand(W)
    prefix = next((p for p in _PREFIXES if p + "embed_tokens.weight" in shards), None)
    if prefix is None:
        raise KeyError(f"{path}: no embed_tokens.weight under {' or '.join(_PREFIXES)}")
    handles = {}

    def get(name):
        f = shards[name]
        if f not in handles:
            handles[f] = safe_open(f, framework="pt")
        return handles[f].get_tensor(name).float()

    W = {}

    def put_linear(key, w, force_q=False):
        if int8 or force_q:
            q, s = quantize_int8(w, group)
            W[key + ".q"], W[key + ".s"] = q, s
        else:
            W[key] = w.contiguous()

    put_linear("embed", get(prefix + "embed_tokens.weight"))
    W["norm"] = get(prefix + "norm.weight")
    if not cfg.tie_embeddings:
        head = "lm_head.weight" if "lm_head.weight" in shards else prefix.replace("model.", "", 1) + "lm_head.weight"
        put_linear("lm_head", get(head))
    for l in range(cfg.layers):
        for key, hname, kind in _layer_names(cfg, l):
            t = get(prefix + hname)
            if kind == "q":
                put_linear(key, t, force_q=key.rsplit(".", 1)[-1] in ("gate_proj", "up_proj", "down_proj"))
            elif kind == "conv":
                W[key] = t.reshape(t.shape[0], t.shape[-1]).contiguous()
            else:
                W[key] = t.contiguous()
    handles.clear()
    if cache_file:
        os.makedirs(cache_dir, exist_ok=True)
        tmp = cache_file + ".tmp"
        save_file({k: v.contiguous() for k, v in W.items()}, tmp, metadata={"format": _CACHE_VERSION})
        os.replace(tmp, cache_file)
    return cfg, _expand(W)
