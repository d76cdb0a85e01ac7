"""ctypes binding of libdyllm_hip.so (the C ABI declared in include/dyllm_hip.h).

There is no fallback: if the library is missing or fails to load, every op raises.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import c_float, c_int, c_int64, c_size_t, c_void_p

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("DYLLM_HIP_LIB") or os.path.join(_HERE, "libdyllm_hip.so")

_P = c_void_p
_I = c_int
_L = c_int64



class KvEpilogue(ctypes.Structure):
    """dyllm_kv_epilogue (include/dyllm_hip.h), field for field."""
    _fields_ = [
        ("kv", c_void_p),
        ("ld_kv", c_int64),
        ("kv_rows", c_void_p),
        ("positions", c_void_p),
        ("pos_idx", c_void_p),
        ("cos_table", c_void_p),
        ("sin_table", c_void_p),
        ("max_position", c_int),
        ("k_norm_weight", c_void_p),
        ("eps", c_float),
        ("k_cache", c_void_p),
        ("k_seq_starts", c_void_p),
    ]


# name -> argtypes (all return int status unless listed in _RET)
SIGNATURES = {
    "dyllm_last_error": [],
    "dyllm_abi_version": [],
    "dyllm_attention_timer": [_I],
    "dyllm_attention_kernel_info": [_I, _I, _P],
    "dyllm_unmask_step": [_P, _P, _I, _P, _P, _P, _L, _P, _P, _P, _P, _L, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                          _P, _I, _P],
    "dyllm_attention_timer_read": [_P, _P],
    "dyllm_issue_probe": [_I, _I, _I, _P, _P, _P],
    "dyllm_attention_sparse_workspace_bytes": [_I, _I, _L, _I],
    "dyllm_attention_sparse_varlen": [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P, _P, _I, _I, _L, _I, _P, _P, _P,
                                      _P, _P, c_float, _P, c_size_t, _P],
    "dyllm_flash_attn_varlen": [_P, _P, _P, _P, _I, _I, _I, _I, _P, _P, _P, _I, _I, c_float, _P, _P],
    "dyllm_attention_colsparse_workspace_bytes": [_I, _I, _L, _L, _I],
    "dyllm_attention_colsparse_cached": [_P, _P, _P, _P, _P, _P, _I, _P, _P, _I, _I, _I, _I, _P, _P, _I, _I, _L,
                                         _L, _I, _P, _P, _P, _P, c_float, _P, c_size_t, _P],
    "dyllm_sparse_step_workspace_bytes": [_I, _I, _I, _I, _L, _L, _I, _L],
    "dyllm_sparse_attention_step": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P, _P, _P, _I, _I, _L, _L,
                                    _I, _I, _P, _P, _P, _P, c_float, c_float, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                    _P, _P, _P, _P, c_size_t, _P],
    "dyllm_sparse_attention_step_kv": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P, _P, _P, _I, _I,
                                       _L, _L, _I, _I, _P, _P, _P, _P, c_float, c_float, _P, _P, _P, _P, _P, _P, _P,
                                       _P, _P, _P, _P, _P, _P, c_size_t, _P],
    "dyllm_sparse_step_scratch_bytes": [],
    "dyllm_sparse_attention_step_noalloc": [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P, _P, _P, _I, _I,
                                            _L, _L, _I, _I, _P, _P, _P, _P, c_float, c_float, _P, _P, _P, _P, _P,
                                            _P, _P, _P, _P, _P, _P, _P, _P],
    "dyllm_v_delta_update": [_P, _P, _P, _L, _L, _P, _P],
    "dyllm_seq_row_starts": [_P, _P, _P, _P, _I, _P, _P],
    "dyllm_cosine_mask": [_P, _L, c_float, _P, _P],
    "dyllm_saliency_stats": [_P, _P, _L, _L, c_float, _P, _P, _P],
    "dyllm_salient_compact": [_P, _L, _P, _I, _P, _P, _P, _P, _P, _P, _P],
    "dyllm_fused_offset_launch": [_P, _P, _P, _P, _I, _P, _L, _P],
    "dyllm_get_seqs": [_P, _P, _L, _P, _P, _P, _I, _L, _P],
    "dyllm_get_block": [_P, _P, _L, _P, _P, _P, _P, _I, _L, _P],
    "dyllm_reset_full": [_P, _P, _L, _P, _P, _P, _I, _L, _P],
    "dyllm_reset_block": [_P, _P, _L, _P, _P, _P, _P, _I, _L, _P],
    "dyllm_scatter_update": [_P, _P, _L, _P, _L, _P, _P, _P, _I, _P],
    "dyllm_scatter_dest_rows": [_P, _L, _P, _P, _P, _P, _I, _P, _P],
    "dyllm_gather_rows": [_P, _L, _P, _L, _P, _L, _P],
    "dyllm_swiglu_ffn_workspace_bytes": [_L, _I],
    "dyllm_swiglu_ffn": [_P, _L, _P, _L, _P, _P, _I, _I, _P, c_size_t, _P, _P, _P],
    "dyllm_silu_and_mul": [_P, _L, _L, _I, _P, _L, _P],
    "dyllm_ffn_tile_rows": [_L, _I, _I, _I],
    "dyllm_ffn_gate_up": [_P, _L, _P, _L, _P, _L, _P, _I, _I, _P, _P],
    "dyllm_ffn_down": [_P, _L, _P, _L, _P, _I, _I, _P, _P, _P, c_size_t, _P],
    "dyllm_ffn_down_workspace_bytes": [_L, _L, _I, _I],
    "dyllm_linear_workspace_bytes": [_L, _L, _I, _I],
    "dyllm_linear": [_P, _L, _P, _L, _P, _L, _P, _I, _I, _P, _P, _P, c_size_t, _P],
    "dyllm_rope": [_P, _L, _L, _I, _I, _P, _P, _P, _I, _P, c_float, _P],
    "dyllm_kv_rope_scatter": [_P, _L, _L, _P, _P, _P, _P, _P, _I, _I, _I, _P, c_float, _P, _P, _P, _P, _P, _I, _P,
                              _P],
    "dyllm_rms_norm": [_P, _L, _P, _L, _P, _L, _I, c_float, _P, _L, _P, _L, _P],
    "dyllm_rms_norm_cache_rows": [_P, _L, _P, _P, _P, _P, _I, _P, _L, _P, _L, _I, c_float, _P, _L, _P, _L, _P],
    "dyllm_moe_gate": [_P, _P, _L, _I, _P, _I, _I, _I, _P, _P, _P],
    "dyllm_moe_align_block_size": [_P, _L, _I, _I, _P, _L, _P, _P, _P],
    "dyllm_fused_experts_workspace_bytes": [_L, _I, _I, _I, _I],
    "dyllm_fused_experts": [_P, _P, _L, _I, _P, _P, _I, _I, _P, _P, _I, _P, _P, _P, c_size_t, _P],
}
_RET = {
    "dyllm_last_error": ctypes.c_char_p,
    "dyllm_abi_version": c_int,
    "dyllm_ffn_tile_rows": c_int,
    "dyllm_attention_sparse_workspace_bytes": c_size_t,
    "dyllm_attention_colsparse_workspace_bytes": c_size_t,
    "dyllm_sparse_step_workspace_bytes": c_size_t,
    "dyllm_sparse_step_scratch_bytes": c_size_t,
    "dyllm_swiglu_ffn_workspace_bytes": c_size_t,
    "dyllm_ffn_down_workspace_bytes": c_size_t,
    "dyllm_linear_workspace_bytes": c_size_t,
    "dyllm_fused_experts_workspace_bytes": c_size_t,
}

_lib = None


def load(path: str = LIB_PATH):
    """Load (once) and return the ctypes handle; raise RuntimeError if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    # torch ships its own libamdhip64 (same SONAME, different file name). Importing torch
    # first makes our DT_NEEDED resolve to that already-loaded runtime; loading ours first
    # would put two HIP runtimes in the process and the second sees no device.
    import torch  # noqa: F401

    if not os.path.exists(path):
        raise RuntimeError(f"libdyllm_hip.so not found at {path}: build it with "
                           f"`python -c 'import __graft_entry__ as g; g.build()'` (no CPU fallback exists)")
    lib = ctypes.CDLL(path)
    for name, args in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = _RET.get(name, c_int)
    _lib = lib
    return lib


def call(name: str, *args):
    """Call an int-status entry point and raise RuntimeError with the library's message."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.dyllm_last_error().decode()
        raise RuntimeError(f"{name}: {msg}")
    return rc
