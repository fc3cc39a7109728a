"""Write tests/golden/qwen35_tiny_golden.safetensors: golden vectors for the layer compositions of the Qwen3.5 hybrid
stack, produced by transformers 5.15.0's own Qwen3_5 modules (models/qwen3_5/modeling_qwen3_5.py, the code the
reference's tests/engine_ref.py runs) on a tiny random configuration.

The weights are not stored: they are regenerated from seeds by tests/golden/tiny_weights.py (q35hip.workloads
init_weights plus random norm gains, so that the (1 + w) and plain-w norm conventions are both exercised) and
loaded into HF's modules here and into the oracle in tests/test_oracle_model.py.

Recorded (all fp32):
  ids                      [2, 70] prompt (crosses one 64-token chunk boundary)
  resid_l{0..3}            residual stream after each decoder layer, every 7th position
  logits_prefill           last-position logits of the 70-token prefill (chunked delta rule, eager attention)
  next_ids, logits_decode  one cached decode step (recurrent delta rule, KV cache) with the prefill's argmax
  logits_steered           prefill with a residual vector added after layer 1 on every position: +v on row 0,
                           -v on row 1 (the forward-hook form of tests/engine_ref.py:49-53)
  acts_l{0..3}             MLP activations (the input of down_proj, recorded by a forward pre-hook as
                           tests/engine_ref.py:11-20 does) of the prefill, every 7th position
  acts_decode_l{0..3}      the same for the cached decode step
  acts_push_l{0..3},       prefill with a neuron push on layer PUSH_LAYER (neuron PUSH_NEURON += PUSH_VALUE on every
  logits_pushed            row and position, the hook's push form of tests/engine_ref.py:14-15): the activations of
                           every layer and the last-position logits

Run from the repository root in the build container (it imports transformers; nothing here runs on a GPU):
    python tests/golden/make_layer_golden.py
"""
import os
import sys

import torch
from safetensors.torch import save_file

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)
sys.path.insert(0, os.path.join(HERE, "..", "..", "duo-mech-interp_amd"))

from tiny_weights import PUSH_LAYER, PUSH_NEURON, PUSH_VALUE, STEER_LAYER, tiny_config, tiny_weights, \
    tiny_inputs  # noqa: E402

from transformers import Qwen3_5TextConfig  # noqa: E402
from transformers.models.qwen3_5.modeling_qwen3_5 import Qwen3_5ForCausalLM  # noqa: E402


def hf_model(cfg, W):
    hcfg = Qwen3_5TextConfig(
        vocab_size=cfg.vocab, hidden_size=cfg.hidden, intermediate_size=cfg.inter, num_hidden_layers=cfg.layers,
        num_attention_heads=cfg.n_heads, num_key_value_heads=cfg.n_kv, head_dim=cfg.head_dim,
        linear_num_key_heads=cfg.lin_k_heads, linear_num_value_heads=cfg.lin_v_heads,
        linear_key_head_dim=cfg.lin_dk, linear_value_head_dim=cfg.lin_dv, linear_conv_kernel_dim=cfg.conv_k,
        rms_norm_eps=cfg.eps, tie_word_embeddings=True,
        rope_parameters={"rope_type": "default", "rope_theta": cfg.rope_theta,
                         "partial_rotary_factor": cfg.partial_rotary})
    hcfg._attn_implementation = "eager"
    m = Qwen3_5ForCausalLM(hcfg).eval()
    sd = {"model.embed_tokens.weight": W["embed"], "model.norm.weight": W["norm"], "lm_head.weight": W["embed"]}
    for l in range(cfg.layers):
        p, hp = f"layers.{l}.", f"model.layers.{l}."
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
    missing, unexpected = m.load_state_dict(sd, strict=False)
    assert not unexpected and not [k for k in missing if "rotary" not in k], (missing, unexpected)
    return m


def main():
    cfg = tiny_config()
    W = tiny_weights(cfg)
    ids, vec = tiny_inputs(cfg)
    m = hf_model(cfg, W)
    out = {"ids": ids}
    resid = {}
    hooks = [m.model.layers[l].register_forward_hook(
        lambda mod, inp, o, l=l: resid.__setitem__(l, (o[0] if isinstance(o, tuple) else o).detach().clone()))
        for l in range(cfg.layers)]
    acts, push = {}, {}

    def pre_hook(l):
        def f(mod, inp):
            h = inp[0]
            if l in push:
                h = h.clone()
                n, v = push[l]
                h[..., n] += v
            acts[l] = h.detach().clone()
            return (h,)
        return f
    hooks += [m.model.layers[l].mlp.down_proj.register_forward_pre_hook(pre_hook(l)) for l in range(cfg.layers)]
    with torch.no_grad():
        r = m(input_ids=ids, use_cache=True)
        for l in range(cfg.layers):
            out[f"acts_l{l}"] = acts[l][:, ::7].contiguous()
        for l in range(cfg.layers):
            out[f"resid_l{l}"] = resid[l][:, ::7].contiguous()
        out["logits_prefill"] = r.logits[:, -1].contiguous()
        nxt = r.logits[:, -1].argmax(-1, keepdim=True)
        out["next_ids"] = nxt
        r2 = m(input_ids=nxt, past_key_values=r.past_key_values, use_cache=True)
        out["logits_decode"] = r2.logits[:, -1].contiguous()
        for l in range(cfg.layers):
            out[f"acts_decode_l{l}"] = acts[l][:, 0].contiguous()
        push[PUSH_LAYER] = (PUSH_NEURON, PUSH_VALUE)
        r4 = m(input_ids=ids)
        push.clear()
        for l in range(cfg.layers):
            out[f"acts_push_l{l}"] = acts[l][:, ::7].contiguous()
        out["logits_pushed"] = r4.logits[:, -1].contiguous()
        for h in hooks:
            h.remove()
        signs = torch.tensor([1.0, -1.0])[:, None, None]
        hv = m.model.layers[STEER_LAYER].register_forward_hook(
            lambda mod, inp, o: ((o[0] + signs * vec,) + tuple(o[1:])) if isinstance(o, tuple) else o + signs * vec)
        r3 = m(input_ids=ids)
        hv.remove()
        out["logits_steered"] = r3.logits[:, -1].contiguous()
    path = os.path.join(HERE, "qwen35_tiny_golden.safetensors")
    save_file({k: v.contiguous() for k, v in out.items()}, path)
    print("wrote", path, {k: tuple(v.shape) for k, v in out.items()})


if __name__ == "__main__":
    main()
