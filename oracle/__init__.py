"""CPU oracle for the Qwen3.5 hybrid-attention hot path.

TEST INFRASTRUCTURE ONLY. This package restates, in plain PyTorch on the CPU (fp32 or fp64), the arithmetic that the
reference's PyTorch mirror (tests/engine_ref.py of scasella/duo-mech-interp) runs through HF transformers 5.15.0
`models/qwen3_5/modeling_qwen3_5.py` (cited as HF:line). Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may import it, and only as the reference that results are compared with or as the timed CPU
baseline; the HIP product never routes through it.

Pinning status of every function is recorded in its module docstring; the checks live in tests/test_oracle_*.py.
"""
from .gdn import l2norm, recurrent_gated_delta_rule, chunk_gated_delta_rule  # noqa: F401
from .attention import (rope_inv_freq, rope_tables, apply_partial_rope, gated_attention,  # noqa: F401
                        gated_attention_decode, gated_attention_cached)
from .steer import residual_steer_add  # noqa: F401
from .metrics import rel_err  # noqa: F401
