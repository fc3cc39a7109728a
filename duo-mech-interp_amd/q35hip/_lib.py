"""ctypes binding of libq35hip.so (the C ABI of include/q35hip.h).

torch is imported first so that the HIP runtime torch ships is the one libq35hip.so binds to (both carry the soname
libamdhip64.so.7; the dynamic linker reuses the already-loaded copy). There is no fallback: if the library is missing
every op raises.
"""
import ctypes
import os

import torch  # noqa: F401  (must precede the library load, see above)

from .build import LIB_PATH

EXPORTS = [
    "q35_status_string", "q35_abi_version",
    "q35_gdn_recurrent", "q35_gdn_chunk_workspace_bytes", "q35_gdn_chunk_prefill",
    "q35_gated_attn_prefill_workspace_bytes", "q35_gated_attn_prefill",
    "q35_gated_attn_prefill_cached_workspace_bytes", "q35_gated_attn_prefill_cached", "q35_gated_attn_decode_workspace_bytes",
    "q35_gated_attn_decode", "q35_gated_attn_decode_noalloc_max_bytes", "q35_gated_attn_decode_noalloc",
    "q35_gated_attn_decode_proj", "q35_gated_attn_prefill_proj_workspace_bytes", "q35_gated_attn_prefill_proj",
    "q35_gated_attn_prefill_cached_proj_workspace_bytes", "q35_gated_attn_prefill_cached_proj",
    "q35_gemv_norm_argmax",
    "q35_resid_add_rows", "q35_gdn_conv", "q35_gdn_decode_fused", "q35_gated_rmsnorm", "q35_attn_prep", "q35_gemv",
    "q35_swiglu_push",
    "q35_add_rmsnorm", "q35_argmax_rows", "q35_gemv_norm", "q35_gemm_q8", "q35_gemm_q8_split",
    "q35_add_rmsnorm_split", "q35_gated_rmsnorm_split", "q35_gemm_q8_bf16",
    "q35_gdn_decode_sliced", "q35_gemv_norm_conv", "q35_gemv_gated_norm", "q35_gdn_chunk_prefill_conv",
]

Q35_F32, Q35_BF16, Q35_I8, Q35_I8_G128 = 0, 1, 2, 3
Q35_ESCRATCH = 5
ABI_VERSION = 14  # the signatures below; q35_abi_version() of the loaded library must match

_lib = None

P = ctypes.c_void_p
I64 = ctypes.c_int64
I32 = ctypes.c_int
F32 = ctypes.c_float
SZ = ctypes.c_size_t

_SIGS = {
    "q35_status_string": ([I32], ctypes.c_char_p),
    "q35_abi_version": ([], I32),
    "q35_gdn_recurrent": ([P, P, P, P, P, P, P, P, I64, I64, I64, I64, I64, I64, I32, F32, I32, P], I32),
    "q35_gdn_chunk_workspace_bytes": ([I64, I64, I64, I64, I64, I64, I32], SZ),
    "q35_gdn_chunk_prefill": ([P, P, P, P, P, P, P, P, I64, I64, I64, I64, I64, I64, I32, F32, I32, I64, P, SZ, P],
                              I32),
    "q35_gated_attn_prefill_workspace_bytes": ([I64, I64, I64, I64, I64], SZ),
    "q35_gated_attn_prefill": ([P, P, P, P, P, P, I64, P, I64, I64, I64, I64, I64, I64, F32, P, SZ, P], I32),
    "q35_gated_attn_prefill_cached_workspace_bytes": ([I64, I64, I64, I64], SZ),
    "q35_gated_attn_prefill_cached": ([P, P, P, P, P, P, P, P, I64, I64, I64, I64, I64, I64, I64, F32, P, SZ, P],
                                      I32),
    "q35_gated_attn_decode_workspace_bytes": ([I64, I64, I64, I64, I64, I64], SZ),
    "q35_gated_attn_decode": ([P, P, P, P, P, P, P, P, I32, I64, I64, I64, I64, I64, I64, F32, I64, P, SZ, P], I32),
    "q35_gated_attn_decode_proj": ([P, I64, P, P, F32, P, P, P, P, P, P, I32, I64, I64, I64, I64, I64, I64, F32, I64,
                                    P, SZ, P], I32),
    "q35_gated_attn_prefill_proj_workspace_bytes": ([I64, I64, I64, I64, I64], SZ),
    "q35_gated_attn_prefill_proj": ([P, I64, P, P, F32, P, P, I64, P, P, P, I64, I64, I64, I64, I64, I64, I64, F32, P,
                                     SZ, P], I32),
    "q35_gated_attn_prefill_cached_proj_workspace_bytes": ([I64, I64, I64, I64, I64, I64], SZ),
    "q35_gated_attn_prefill_cached_proj": ([P, I64, P, P, F32, P, P, P, P, P, P, I64, I64, I64, I64, I64, I64, I64, F32,
                                            P, SZ, P], I32),
    "q35_gated_attn_decode_noalloc_max_bytes": ([], SZ),
    "q35_gated_attn_decode_noalloc": ([P, P, P, P, P, P, P, P, I32, I64, I64, I64, I64, I64, I64, F32, I64, P], I32),
    "q35_resid_add_rows": ([P, P, P, I64, I64, I64, I64, I32, P], I32),
    "q35_gdn_conv": ([P, I64, P, P, P, P, P, I64, I64, P, P, P, P, P, I64, I64, I64, I64, I64, I64, I64, I32, P], I32),
    "q35_gdn_chunk_prefill_conv": ([P, I64, P, P, P, P, P, I64, I64, P, P, P, I64, I64, I64, I64, I64, I64, I64, F32,
                                    P, SZ, P], I32),
    "q35_gated_rmsnorm": ([P, P, I64, P, P, P, I64, I64, I64, F32, I32, P], I32),
    "q35_gated_rmsnorm_split": ([P, P, I64, P, P, P, I64, I64, I64, F32, P], I32),
    "q35_gdn_decode_fused": ([P, I64, P, P, P, P, P, I64, I64, I64, P, P, P, F32, F32, P, I64, I64, I64, I64, P],
                             I32),
    "q35_attn_prep": ([P, I64, P, P, F32, P, P, I64, P, P, P, P, P, P, P, I64, I64, I64, I64, I64, I64, P], I32),
    "q35_gemv": ([P, I64, P, I32, P, P, I64, I64, I64, I64, I32, P, I64, I64, P, I64, I64, P], I32),
    "q35_swiglu_push": ([P, P, I64, I64, P, I64, I64, P, I64, I64, P], I32),
    "q35_add_rmsnorm": ([P, I64, P, I64, P, P, I64, I64, I64, F32, P], I32),
    "q35_add_rmsnorm_split": ([P, I64, P, I64, P, P, I64, I64, I64, F32, P], I32),
    "q35_argmax_rows": ([P, I64, I64, I64, P, P, P], I32),
    "q35_gemm_q8": ([P, I64, P, I32, P, P, I64, I64, I64, I64, I32, P, I64, I64, P, I64, I64, P], I32),
    "q35_gemm_q8_split": ([P, I64, P, I32, P, P, I64, I64, I64, I64, I32, P, I64, I64, P, I64, I64, P], I32),
    "q35_gemm_q8_bf16": ([P, I64, P, I32, P, P, I64, I64, I64, I64, I32, P, I64, I64, P, I64, I64, P], I32),
    "q35_gemv_norm": ([P, P, P, I64, P, F32, P, I32, P, P, I64, I64, I64, I64, I32, P, I64, I64, P, I64, I64, P],
                      I32),
    "q35_gemv_norm_argmax": ([P, P, P, I64, P, F32, P, I32, P, P, I64, I64, I64, I64, P, P, P], I32),
    "q35_gdn_decode_sliced": ([P, I64, P, P, I64, I64, P, F32, P, I64, I64, I64, P], I32),
    "q35_gemv_norm_conv": ([P, P, P, I64, P, F32, P, I32, P, P, I64, I64, I64, I64, P, P, P, I64, I64, P], I32),
    "q35_gemv_gated_norm": ([P, I64, P, I64, P, P, F32, P, I32, P, P, I64, I64, I64, I64, I32, P], I32),
}


class Q35Error(RuntimeError):
    pass


def lib():
    """The loaded library (loaded on first use). Raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise Q35Error(f"q35hip: {LIB_PATH} is missing; build it with __graft_entry__.build() "
                           "(python -m q35hip.build). There is no CPU fallback.")
        L = ctypes.CDLL(LIB_PATH)
        L.q35_abi_version.restype = I32
        found = L.q35_abi_version()
        if found != ABI_VERSION:
            raise Q35Error(f"q35hip: {LIB_PATH} has ABI version {found}, this package binds version {ABI_VERSION}; "
                           "rebuild it with __graft_entry__.build() (python -m q35hip.build)")
        for name, (argt, rest) in _SIGS.items():
            fn = getattr(L, name)
            fn.argtypes = argt
            fn.restype = rest
        _lib = L
    return _lib


def check(status, what):
    if status != 0:
        msg = lib().q35_status_string(status).decode()
        raise Q35Error(f"q35hip: {what} failed with status {status} ({msg})")
