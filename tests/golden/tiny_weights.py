"""Seeded weights and inputs of the tiny Qwen3.5 configuration used by the golden vectors
(tests/golden/qwen35_tiny_golden.safetensors): shared by the fixture writer and the tests, so that the fixture
stores only inputs and outputs."""
import torch

from q35hip.workloads import Q35Config, init_weights

STEER_LAYER = 1
PUSH_LAYER, PUSH_NEURON, PUSH_VALUE = 2, 5, 0.75  # the neuron push of the fixture's pushed prefill


def tiny_config():
    return Q35Config(vocab=256, hidden=128, inter=256, layers=4, n_heads=2, n_kv=1, head_dim=256, lin_k_heads=2,
                     lin_v_heads=2, lin_dk=128, lin_dv=128)


def tiny_weights(cfg):
    """init_weights(seed 1) with random norm gains (seed 2): the decoder / q / k RMSNorms use (1 + w), the gated
    norm plain w, and both must show up in the outputs."""
    # the weights the golden vectors were written with: fp32 mixers, MLP int8 with one scale per row
    W = init_weights(cfg, seed=1, int8_all=False, group=0)
    g = torch.Generator().manual_seed(2)
    for k in sorted(W):
        if k.endswith("layernorm") or k.endswith("q_norm") or k.endswith("k_norm") or k == "norm":
            W[k] = 0.3 * torch.randn(W[k].shape, generator=g)
        elif k.endswith(".norm"):
            W[k] = 1.0 + 0.3 * torch.randn(W[k].shape, generator=g)
    # larger linear weights than the 0.02 default, so that every mixer contributes visibly to the residual
    for k in sorted(W):
        if any(k.endswith(n) for n in ("in_proj_qkv", "in_proj_z", "out_proj", "q_proj", "k_proj", "v_proj",
                                       "o_proj", "conv1d", "in_proj_b", "in_proj_a")):
            W[k] = W[k] * 5.0
    return W


def tiny_inputs(cfg):
    g = torch.Generator().manual_seed(3)
    ids = torch.randint(0, cfg.vocab, (2, 70), generator=g)
    vec = 0.5 * torch.randn(cfg.hidden, generator=g)
    return ids, vec
