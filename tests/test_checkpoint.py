"""Local checkpoint loading (q35hip.checkpoint): a tiny HF-layout checkpoint (config.json + bf16 safetensors under the
multimodal "model.language_model." prefix, engine/model.js:21-23) written here from the seeded tiny weights, loaded
back, compared tensor by tensor, through a sharded index and the int8 cache, and run through the oracle. CPU only."""
import json
import os
import sys

import torch
from safetensors.torch import save_file

from oracle import model as om
from q35hip import checkpoint as ck
from q35hip.workloads import Q35Config, quantize_groups_int8, quantize_rows_int8

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))
from tiny_weights import tiny_config, tiny_inputs, tiny_weights  # noqa: E402

PREFIX = "model.language_model."


def _bf(t):
    return t.to(torch.bfloat16).float()


def _hf_tensors(cfg, W):
    """HF names (HF:426-429, :641-654) -> bf16 tensors of the tiny weights (the MLP dequantised)."""
    sd = {PREFIX + "embed_tokens.weight": W["embed"], PREFIX + "norm.weight": W["norm"]}
    for l in range(cfg.layers):
        p, hp = f"layers.{l}.", f"{PREFIX}layers.{l}."
        sd[hp + "input_layernorm.weight"] = W[p + "input_layernorm"]
        sd[hp + "post_attention_layernorm.weight"] = W[p + "post_attention_layernorm"]
        for n in ("gate_proj", "up_proj", "down_proj"):
            sd[hp + f"mlp.{n}.weight"] = W[p + n + ".q"].float() * W[p + n + ".s"][:, None]
        if cfg.is_attention(l):
            for n in ("q_proj", "k_proj", "v_proj", "o_proj", "q_norm", "k_norm"):
                sd[hp + f"self_attn.{n}.weight"] = W[p + n]
        else:
            for n in ("in_proj_qkv", "in_proj_z", "in_proj_b", "in_proj_a", "out_proj", "norm"):
                sd[hp + f"linear_attn.{n}.weight"] = W[p + n]
            sd[hp + "linear_attn.conv1d.weight"] = W[p + "conv1d"][:, None, :]
            sd[hp + "linear_attn.dt_bias"] = W[p + "dt_bias"]
            sd[hp + "linear_attn.A_log"] = W[p + "A_log"]
    return {k: v.to(torch.bfloat16).contiguous() for k, v in sd.items()}


def _hf_config(cfg):
    text = dict(vocab_size=cfg.vocab, hidden_size=cfg.hidden, intermediate_size=cfg.inter,
                num_hidden_layers=cfg.layers, num_attention_heads=cfg.n_heads, num_key_value_heads=cfg.n_kv,
                head_dim=cfg.head_dim, linear_num_key_heads=cfg.lin_k_heads, linear_num_value_heads=cfg.lin_v_heads,
                linear_key_head_dim=cfg.lin_dk, linear_value_head_dim=cfg.lin_dv,
                linear_conv_kernel_dim=cfg.conv_k, rms_norm_eps=cfg.eps, tie_word_embeddings=True,
                layer_types=["full_attention" if cfg.is_attention(l) else "linear_attention"
                             for l in range(cfg.layers)],
                rope_parameters={"rope_type": "default", "rope_theta": cfg.rope_theta,
                                 "partial_rotary_factor": cfg.partial_rotary})
    return {"model_type": "qwen3_5", "text_config": text, "tie_word_embeddings": True}


def _write(path, cfg, W, shards=1):
    os.makedirs(path, exist_ok=True)
    json.dump(_hf_config(cfg), open(os.path.join(path, "config.json"), "w"))
    sd = _hf_tensors(cfg, W)
    if shards == 1:
        save_file(sd, os.path.join(path, "model.safetensors"))
        return sd
    names = sorted(sd)
    wm = {}
    for i in range(shards):
        part = names[i::shards]
        f = f"model-{i + 1:05d}-of-{shards:05d}.safetensors"
        save_file({k: sd[k] for k in part}, os.path.join(path, f))
        wm.update({k: f for k in part})
    json.dump({"weight_map": wm}, open(os.path.join(path, "model.safetensors.index.json"), "w"))
    return sd


def test_config_from_hf_reads_the_text_config():
    cfg = tiny_config()
    got = ck.config_from_hf(_hf_config(cfg))
    for f in ("vocab", "hidden", "inter", "layers", "n_heads", "n_kv", "head_dim", "lin_k_heads", "lin_v_heads",
              "lin_dk", "lin_dv", "conv_k", "rope_theta", "partial_rotary", "eps"):
        assert getattr(got, f) == getattr(cfg, f), f
    assert [got.is_attention(l) for l in range(cfg.layers)] == [cfg.is_attention(l) for l in range(cfg.layers)]
    # a text-only config without the nesting, with the interval form of the layer pattern
    flat = dict(_hf_config(cfg)["text_config"])
    del flat["layer_types"]
    flat["full_attention_interval"] = 2
    got = ck.config_from_hf(flat)
    assert [got.is_attention(l) for l in range(4)] == [False, True, False, True]


def test_load_fp32_matches_the_bf16_tensors(tmp_path):
    cfg = tiny_config()
    W0 = tiny_weights(cfg)
    sd = _write(str(tmp_path / "ckpt"), cfg, W0)
    c2, W = ck.load_checkpoint(str(tmp_path / "ckpt"), int8=False, cache_dir=False)
    assert torch.equal(W["embed"], sd[PREFIX + "embed_tokens.weight"].float())
    p = "layers.0."
    assert torch.equal(W[p + "in_proj_qkv"], sd[PREFIX + p + "linear_attn.in_proj_qkv.weight"].float())
    assert tuple(W[p + "conv1d"].shape) == (W0[p + "conv1d"].shape[0], cfg.conv_k)
    assert torch.equal(W[p + "conv1d"], _bf(W0[p + "conv1d"]))
    q, s = quantize_groups_int8(sd[PREFIX + p + "mlp.down_proj.weight"].float())
    assert torch.equal(W[p + "down_proj.q"], q) and torch.equal(W[p + "down_proj.s"], s)
    l_att = next(l for l in range(cfg.layers) if cfg.is_attention(l))
    assert torch.equal(W[f"layers.{l_att}.q_norm"], _bf(W0[f"layers.{l_att}.q_norm"]))


def test_load_int8_sharded_and_cached_gives_one_dict(tmp_path):
    cfg = tiny_config()
    W0 = tiny_weights(cfg)
    sd = _write(str(tmp_path / "one"), cfg, W0)
    _write(str(tmp_path / "three"), cfg, W0, shards=3)
    _, Wa = ck.load_checkpoint(str(tmp_path / "one"), cache_dir=False)
    _, Wb = ck.load_checkpoint(str(tmp_path / "three"))           # writes the cache
    assert os.listdir(str(tmp_path / "three" / ".q35cache"))
    _, Wc = ck.load_checkpoint(str(tmp_path / "three"))           # reads it
    assert sorted(Wa) == sorted(Wb) == sorted(Wc)
    for k in Wa:
        assert torch.equal(Wa[k], Wb[k]) and torch.equal(Wb[k], Wc[k]), k
    p = "layers.0."
    w = sd[PREFIX + p + "linear_attn.out_proj.weight"].float()
    q, s = quantize_groups_int8(w)                                   # the engine's q8: a scale per 128 inputs
    assert torch.equal(Wa[p + "out_proj.q"], q) and torch.equal(Wa[p + "out_proj.s"], s)
    assert tuple(s.shape) == (w.shape[0], w.shape[1] // 128)
    exp = (q.float().reshape(w.shape[0], -1, 128) * s[:, :, None]).reshape(w.shape)
    assert torch.equal(Wa[p + "out_proj"], exp)                       # the dequantised copy beside it
    assert "layers.0.gate_proj" not in Wa                            # the MLP stays int8 only
    assert Wa["embed.q"].dtype == torch.int8
    # per-row scales on request, cached apart from the per-group form
    _, Wr = ck.load_checkpoint(str(tmp_path / "three"), group=0)
    q, s = quantize_rows_int8(w)
    assert torch.equal(Wr[p + "out_proj.q"], q) and torch.equal(Wr[p + "out_proj.s"], s)
    assert len(os.listdir(str(tmp_path / "three" / ".q35cache"))) == 2


def test_oracle_runs_the_loaded_checkpoint(tmp_path):
    """The loaded fp32 checkpoint gives the oracle's logits of the bf16-rounded weights exactly."""
    cfg = tiny_config()
    W0 = tiny_weights(cfg)
    _write(str(tmp_path / "ckpt"), cfg, W0)
    c2, W = ck.load_checkpoint(str(tmp_path / "ckpt"), int8=False, cache_dir=False)
    Wr = {}
    for k, v in W0.items():
        if k.endswith(".q") or k.endswith(".s"):
            continue
        Wr[k] = _bf(v)
    for l in range(cfg.layers):
        for n in ("gate_proj", "up_proj", "down_proj"):
            b = f"layers.{l}.{n}"
            q, s = quantize_groups_int8(_bf(W0[b + ".q"].float() * W0[b + ".s"][:, None]))
            Wr[b + ".q"], Wr[b + ".s"] = q, s
    ids, _ = tiny_inputs(cfg)
    la, _ = om.OracleModel(c2, W).forward(ids[:, :20])
    lb, _ = om.OracleModel(cfg, Wr).forward(ids[:, :20])
    assert torch.equal(la, lb)
