"""q35hip: MI355X (gfx950) kernels for the Qwen3.5 hybrid-attention hot path, behind torch.library ops.

Importing the package registers the q35:: ops; the HIP library itself is loaded on first use (and raises if it has
not been built: there is no CPU fallback).
"""
from ._lib import Q35Error, lib  # noqa: F401
from .ops import (chunk_gated_delta_rule, gated_attention_decode, gated_attention_prefill,  # noqa: F401
                  gdn_decode_step_, recurrent_gated_delta_rule, residual_steer_add_)

__all__ = ["Q35Error", "lib", "chunk_gated_delta_rule", "recurrent_gated_delta_rule", "gdn_decode_step_",
           "gated_attention_prefill", "gated_attention_decode", "residual_steer_add_"]
