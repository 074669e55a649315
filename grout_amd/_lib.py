"""ctypes bindings of libgrout_attn_hip.so (include/grout_attn_hip.h).

The library is the product; this module only declares argument types.  Loading
fails loudly when the library has not been built: there is no fallback path.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libgrout_attn_hip.so")

c_i32 = ctypes.c_int32
c_u32 = ctypes.c_uint32
c_u16 = ctypes.c_uint16
c_f32 = ctypes.c_float
c_i64 = ctypes.c_int64
c_vp = ctypes.c_void_p

GROUT_OK = 0
STATUS_NAMES = {
    0: "GROUT_OK",
    -1: "GROUT_ERR_NULL_POINTER",
    -2: "GROUT_ERR_ALIGNMENT",
    -3: "GROUT_ERR_HEAD_DIM",
    -4: "GROUT_ERR_HEADS",
    -5: "GROUT_ERR_SEQ_RANGE",
    -6: "GROUT_ERR_KV_LEN",
    -7: "GROUT_ERR_GROUP",
    -8: "GROUT_ERR_SPLITS",
    -9: "GROUT_ERR_ARG",
    -10: "GROUT_ERR_GRAPH",
    -11: "GROUT_ERR_SCRATCH",
}
NAME_TO_STATUS = {v: k for k, v in STATUS_NAMES.items()}


class DecodeLayer(ctypes.Structure):
    """struct grout_decode_layer."""
    _fields_ = [
        ("qkv", c_vp), ("q_weight", c_vp), ("k_weight", c_vp), ("inv_freq", c_vp),
        ("q_out", c_vp), ("k_cache", c_vp), ("v_cache", c_vp), ("att_partial", c_vp),
        ("lse_partial", c_vp), ("attn_out", c_vp), ("d_position", c_vp),
        ("counters", c_vp), ("eps", c_f32), ("qk_scale_f16", c_u16), ("num_q_heads", c_i32),
        ("num_kv_heads", c_i32), ("head_dim", c_i32), ("max_seq_len", c_i32),
        ("block_n", c_i32), ("num_splits", c_i32),
    ]


class Qwen3Layer(ctypes.Structure):
    """struct grout_qwen3_layer."""
    _fields_ = [
        ("input_norm", c_vp), ("qkv_proj", c_vp), ("q_norm", c_vp), ("k_norm", c_vp),
        ("o_proj", c_vp), ("post_attn_norm", c_vp), ("gate_up_proj", c_vp),
        ("down_proj", c_vp), ("k_cache", c_vp), ("v_cache", c_vp),
    ]


class Qwen3Model(ctypes.Structure):
    """struct grout_qwen3_model."""
    _fields_ = [
        ("num_layers", c_i32), ("hidden", c_i32), ("intermediate", c_i32), ("vocab", c_i32),
        ("num_q_heads", c_i32), ("num_kv_heads", c_i32), ("head_dim", c_i32),
        ("max_seq_len", c_i32), ("block_n", c_i32), ("num_splits", c_i32), ("eps", c_f32),
        ("qk_scale_f16", c_u16), ("layers", ctypes.POINTER(Qwen3Layer)),
        ("embed_tokens", c_vp), ("final_norm", c_vp), ("lm_head", c_vp), ("inv_freq", c_vp),
        ("token", c_vp), ("d_position", c_vp), ("logits", c_vp), ("workspace", c_vp),
    ]


# name -> (restype, argtypes)
SIGNATURES = {
    "grout_status_string": (ctypes.c_char_p, [c_i32]),
    "grout_build_inv_freq": (c_i32, [c_f32, c_i32, ctypes.POINTER(c_f32)]),
    "grout_qk_norm_rope_kv_prefill": (
        c_i32, [c_vp] * 9 + [c_f32] + [c_i32] * 6 + [c_vp]),
    "grout_qk_norm_rope_kv_decode": (
        c_i32, [c_vp] * 8 + [c_f32] + [c_i32] * 4 + [c_vp]),
    "grout_attn_prefill": (c_i32, [c_vp] * 4 + [c_f32] + [c_i32] * 7 + [c_vp]),
    "grout_attn_prefill_sched": (c_i32, [c_vp] * 4 + [c_f32] + [c_i32] * 7 + [c_vp, c_vp]),
    "grout_attn_prefill_sched_counter_bytes": (c_i64, []),
    "grout_attn_prefill_split": (c_i32, [c_vp] * 5 + [c_f32] + [c_i32] * 11 + [c_vp]),
    "grout_attn_prefill_split_merge": (c_i32, [c_vp] * 3 + [c_i32] * 6 + [c_vp]),
    "grout_attn_prefill_split_partial_bytes": (c_i64, [c_i32] * 6),
    "grout_attn_prefill_split_lse_bytes": (c_i64, [c_i32] * 5),
    "grout_add_rms_norm_decode": (c_i32, [c_vp] * 5 + [c_f32, c_i32, c_vp]),
    "grout_gemv_f16": (c_i32, [c_vp] * 3 + [c_i32] * 2 + [c_vp]),
    "grout_gemv_silu_mul_f16": (c_i32, [c_vp] * 3 + [c_i32] * 2 + [c_vp]),
    "grout_argmax_blocks": (c_i32, [c_i32]),
    "grout_argmax_f16": (c_i32, [c_vp] * 4 + [c_i32, c_vp]),
    "grout_embed_rms_norm_decode": (c_i32, [c_vp, c_vp, c_i32, c_vp, c_vp, c_vp, c_f32, c_i32,
                                            c_vp]),
    "grout_silu_mul_f16": (c_i32, [c_vp] * 3 + [c_i32, c_vp]),
    "grout_cast_to_f16": (c_i32, [c_vp, c_i32, c_vp, c_i64, c_vp]),
    "grout_qwen3_workspace_bytes": (c_i64, [ctypes.POINTER(Qwen3Model)]),
    "grout_qwen3_decode_step": (c_i32, [ctypes.POINTER(Qwen3Model), c_vp]),
    "grout_qwen3_runner_create": (
        c_i32, [ctypes.POINTER(Qwen3Model), c_u32, c_vp, ctypes.POINTER(c_vp)]),
    "grout_qwen3_runner_seed_token": (c_i32, [c_vp, c_u32]),
    "grout_qwen3_runner_step": (c_i32, [c_vp, c_u32, ctypes.POINTER(c_u32)]),
    "grout_qwen3_runner_run": (c_i32, [c_vp, c_u32, c_i32]),
    "grout_qwen3_runner_destroy": (c_i32, [c_vp]),
    "grout_attn_decode_split": (
        c_i32, [c_vp] * 5 + [c_u16, c_vp] + [c_i32] * 6 + [c_vp]),
    "grout_attn_decode_merge": (c_i32, [c_vp] * 3 + [c_i32] * 4 + [c_vp]),
    "grout_attn_decode_fused": (
        c_i32, [c_vp] * 12 + [c_f32, c_u16] + [c_i32] * 7 + [c_vp]),
    "grout_attn_decode_fused_noalloc": (
        c_i32, [c_vp] * 9 + [c_f32, c_u16] + [c_i32] * 7 + [c_vp]),
    "grout_attn_decode_counter_bytes": (c_i64, [c_i32]),
    "grout_attn_decode_partial_bytes": (c_i64, [c_i32] * 4),
    "grout_attn_decode_lse_bytes": (c_i64, [c_i32] * 3),
    "grout_attn_decode_pick_splits": (c_i32, [c_i32] * 4),
    "grout_attn_decode_pick_splits_grouped": (c_i32, [c_i32] * 5),
    "grout_device_cu_count": (c_i32, [c_i32, ctypes.POINTER(c_i32)]),
    "grout_graph_begin": (c_i32, [c_vp]),
    "grout_graph_end": (c_i32, [c_vp, ctypes.POINTER(c_vp)]),
    "grout_graph_launch": (c_i32, [c_vp, c_vp]),
    "grout_graph_destroy": (c_i32, [c_vp]),
    "grout_set_position_async": (c_i32, [c_vp, c_u32, c_vp]),
    "grout_decode_runner_create": (
        c_i32, [ctypes.POINTER(DecodeLayer), c_u32, c_vp, ctypes.POINTER(c_vp)]),
    "grout_kv_cache_update_seq": (c_i32, [c_vp] * 4 + [c_i32] * 5 + [c_vp]),
    "grout_kv_cache_update_seq_dynpos": (c_i32, [c_vp] * 5 + [c_i32] * 4 + [c_vp]),
    "grout_decode_runner_step": (c_i32, [c_vp, c_u32]),
    "grout_decode_runner_run": (c_i32, [c_vp, c_u32, c_i32]),
    "grout_decode_runner_zero_kv": (c_i32, [c_vp]),
    "grout_decode_runner_destroy": (c_i32, [c_vp]),
}

_lib = None


class LibraryMissing(RuntimeError):
    pass


def load(path: str | None = None):
    """Load (once) and return the ctypes handle of libgrout_attn_hip.so."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = path or LIB_PATH
    if not os.path.exists(p):
        raise LibraryMissing(
            f"{p} is not built; run `python -m grout_amd.build` (there is no CPU fallback)")
    lib = ctypes.CDLL(p)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if path is None:
        _lib = lib
    return lib
