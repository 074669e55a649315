"""ctypes wrapper of the CPU oracle (oracle/grout_oracle.c).

TEST INFRASTRUCTURE ONLY.  Imported by tests/, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py`` as the checker / CPU baseline; the
product (``grout_amd``) never imports it.

Arrays are numpy: f16 tensors travel as ``np.float16`` (bit patterns are passed
to C as uint16), f32 as ``np.float32``.  Every function restates a reference
function; the C file cites the reference file:line for each.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_u16p = ctypes.POINTER(ctypes.c_uint16)
_f32p = ctypes.POINTER(ctypes.c_float)
_i32 = ctypes.c_int32


def build(force: bool = False) -> str:
    """Compile oracle/liboracle.so with the committed Makefile."""
    if force or not os.path.exists(_LIB_PATH):
        cmd = ["make", "-s", "-C", _HERE] + (["-B"] if force else [])
        subprocess.run(cmd, check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.go_f32_to_f16.restype = ctypes.c_uint16
        L.go_f32_to_f16.argtypes = [ctypes.c_float]
        L.go_f16_to_f32.restype = ctypes.c_float
        L.go_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.go_f32_to_f16_array.argtypes = [_f32p, _u16p, ctypes.c_int64]
        L.go_f16_to_f32_array.argtypes = [_u16p, _f32p, ctypes.c_int64]
        L.go_build_inv_freq.argtypes = [ctypes.c_float, _i32, _f32p]
        L.go_qk_norm_rope_kv_prefill.argtypes = (
            [_u16p] * 5 + [_f32p] + [_u16p] * 3 + [ctypes.c_float] + [_i32] * 6)
        L.go_qk_norm_rope_kv_decode.argtypes = (
            [_u16p] * 3 + [_f32p] + [_u16p] * 3 + [ctypes.c_uint32, ctypes.c_float]
            + [_i32] * 4)
        L.go_attn_prefill_f32.argtypes = (
            [_u16p] * 3 + [_f32p, ctypes.c_float] + [_i32] * 10)
        L.go_attn_decode_split.argtypes = (
            [_u16p] * 4 + [_f32p, ctypes.c_uint16, ctypes.c_uint32] + [_i32] * 8)
        L.go_decode_split_range_fused.argtypes = [_i32] * 3 + [ctypes.POINTER(_i32)] * 2
        L.go_attn_decode_merge.argtypes = [_u16p, _f32p, _u16p] + [_i32] * 4
        L.go_decode_split_range.argtypes = [_i32] * 4 + [ctypes.POINTER(_i32)] * 2
        L.go_kv_cache_update_seq.argtypes = [_u16p] * 4 + [_i32] * 5
        L.go_attn_prefill_split.argtypes = (
            [_u16p] * 4 + [_f32p, ctypes.c_float] + [_i32] * 12)
        L.go_attn_prefill_split_merge.argtypes = [_u16p, _f32p, _u16p] + [_i32] * 6
        L.go_add_rms_norm.argtypes = [_u16p] * 5 + [ctypes.c_float, _i32]
        L.go_gemv_f16.argtypes = [_u16p] * 3 + [_i32] * 3
        L.go_argmax_f16.restype = ctypes.c_uint32
        L.go_argmax_f16.argtypes = [_u16p, _i32]
        L.go_silu_mul.argtypes = [_u16p] * 3 + [_i32]
        L.go_cast_to_f16.restype = _i32
        L.go_cast_to_f16.argtypes = [ctypes.c_void_p, _i32, _u16p, ctypes.c_int64]
        _lib = L
    return _lib


def _u16(a: np.ndarray):
    assert a.dtype == np.float16 and a.flags.c_contiguous, (a.dtype, a.flags)
    return a.ctypes.data_as(_u16p)


def _f32(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous, (a.dtype, a.flags)
    return a.ctypes.data_as(_f32p)


# ------------------------------------------------------------------ f16 ----

def f32_to_f16(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.float16)
    lib().go_f32_to_f16_array(_f32(x), _u16(out), x.size)
    return out


def f16_to_f32(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float16)
    out = np.empty(x.shape, dtype=np.float32)
    lib().go_f16_to_f32_array(_u16(x), _f32(out), x.size)
    return out


def f16_bits(x: float) -> int:
    """f16 bit pattern of f32(x), as src/model.rs:3427 f16::from_f32(qk_scale)."""
    return int(lib().go_f32_to_f16(float(np.float32(x))))


# ---------------------------------------------------------------- kernels --

def build_inv_freq(theta: float, head_dim: int = 128) -> np.ndarray:
    out = np.empty(head_dim // 2, dtype=np.float32)
    lib().go_build_inv_freq(float(np.float32(theta)), head_dim, _f32(out))
    return out


def qk_norm_rope_kv_prefill(q, k, v, q_weight, k_weight, inv_freq, k_cache, v_cache,
                            eps: float, position_start: int):
    """Returns q_out; writes k_cache / v_cache in place (like the kernel)."""
    S, Hq, D = q.shape
    Hkv = k.shape[1]
    max_seq = k_cache.shape[1]
    q_out = np.zeros_like(q)
    lib().go_qk_norm_rope_kv_prefill(
        _u16(q), _u16(k), _u16(v), _u16(q_weight), _u16(k_weight), _f32(inv_freq),
        _u16(q_out), _u16(k_cache), _u16(v_cache), float(eps), position_start, S, Hq, Hkv,
        D, max_seq)
    return q_out


def qk_norm_rope_kv_decode(qkv, q_weight, k_weight, inv_freq, q_out, k_cache, v_cache,
                           position: int, eps: float, num_q_heads: int, num_kv_heads: int):
    D = q_weight.shape[0]
    max_seq = k_cache.shape[1]
    lib().go_qk_norm_rope_kv_decode(
        _u16(qkv), _u16(q_weight), _u16(k_weight), _f32(inv_freq), _u16(q_out),
        _u16(k_cache), _u16(v_cache), position, float(eps), num_q_heads, num_kv_heads, D,
        max_seq)


def attn_prefill_f32(q, k_cache, v_cache, qk_scale: float, kv_len: int, query_start: int,
                     row_begin: int = 0, row_step: int = 1, nthreads: int = 0,
                     out: np.ndarray | None = None) -> np.ndarray:
    S, Hq, D = q.shape
    Hkv, max_seq, _ = k_cache.shape
    if out is None:
        out = np.zeros((S, Hq, D), dtype=np.float32)
    lib().go_attn_prefill_f32(
        _u16(q), _u16(k_cache), _u16(v_cache), _f32(out), float(qk_scale), Hq, Hkv, D, S,
        kv_len, query_start, max_seq, row_begin, row_step, nthreads)
    return out


def attn_decode_split(q, k_cache, v_cache, qk_scale_f16_bits: int, position: int,
                      block_n: int, num_splits: int, nthreads: int = 0,
                      fused_ranges: bool = False):
    """q [Hkv, G, D] f16 -> (att_partial [Hkv, NKS*G, D] f16, lse [Hkv, NKS*G] f32).
    fused_ranges: the split boundaries of the fused decode step
    (decode_split_range_fused) instead of the reference's."""
    Hkv, G, D = q.shape
    max_seq = k_cache.shape[1]
    att = np.zeros((Hkv, num_splits * G, D), dtype=np.float16)
    lse = np.zeros((Hkv, num_splits * G), dtype=np.float32)
    lib().go_attn_decode_split(
        _u16(q), _u16(k_cache), _u16(v_cache), _u16(att), _f32(lse), qk_scale_f16_bits,
        position, Hkv, G, D, max_seq, block_n, num_splits, nthreads, int(bool(fused_ranges)))
    return att, lse


def attn_decode_merge(att, lse, group: int) -> np.ndarray:
    Hkv, nsg, D = att.shape
    ns = nsg // group
    out = np.zeros((Hkv, group, D), dtype=np.float16)
    lib().go_attn_decode_merge(_u16(att), _f32(lse), _u16(out), Hkv, group, D, ns)
    return out


def decode_split_range_fused(s_kv: int, num_splits: int, split: int):
    """Token range [b, e) of a split in the fused decode step (balanced 16-token
    sub-chunks; this repository's choice, not the reference's)."""
    b, e = _i32(), _i32()
    lib().go_decode_split_range_fused(s_kv, num_splits, split, ctypes.byref(b), ctypes.byref(e))
    return b.value, e.value


def decode_split_range(s_kv: int, block_n: int, num_splits: int, split: int):
    b, e = _i32(), _i32()
    lib().go_decode_split_range(s_kv, block_n, num_splits, split, ctypes.byref(b),
                                ctypes.byref(e))
    return b.value, e.value


def kv_cache_update_seq(new_k, new_v, k_cache, v_cache, position_start: int):
    """Writes cache rows [position_start, position_start+S) in place."""
    S, Hkv, D = new_k.shape
    lib().go_kv_cache_update_seq(_u16(new_k), _u16(new_v), _u16(k_cache), _u16(v_cache),
                                 position_start, S, Hkv, D, k_cache.shape[1])


def attn_prefill_split(q, k_cache, v_cache, qk_scale: float, kv_len: int, query_start: int,
                       block_m: int, block_n: int, group: int, num_splits: int,
                       nthreads: int = 0):
    """q [S, Hq, D] -> (att_partial [tiles, NKS*BM*group, D] f16, lse [tiles, NKS*BM*group])."""
    S, Hq, D = q.shape
    Hkv, max_seq, _ = k_cache.shape
    tiles = -(-S // block_m) * (Hq // group)
    ns_m = num_splits * block_m * group
    att = np.zeros((tiles, ns_m, D), dtype=np.float16)
    lse = np.zeros((tiles, ns_m), dtype=np.float32)
    lib().go_attn_prefill_split(
        _u16(q), _u16(k_cache), _u16(v_cache), _u16(att), _f32(lse), float(qk_scale), Hq, Hkv,
        D, S, kv_len, query_start, max_seq, block_m, block_n, group, num_splits, nthreads)
    return att, lse


def attn_prefill_split_merge(att, lse, num_q_heads: int, q_len: int, block_m: int, group: int,
                             num_splits: int) -> np.ndarray:
    D = att.shape[2]
    out = np.zeros((q_len, num_q_heads, D), dtype=np.float16)
    lib().go_attn_prefill_split_merge(_u16(att), _f32(lse), _u16(out), num_q_heads, D, q_len,
                                      block_m, group, num_splits)
    return out


def add_rms_norm(residual, x, w, eps: float):
    """-> (out, residual_out), f16 [n] each."""
    n = residual.shape[0]
    out = np.zeros(n, dtype=np.float16)
    res = np.zeros(n, dtype=np.float16)
    lib().go_add_rms_norm(_u16(residual), _u16(x), _u16(w), _u16(out), _u16(res), float(eps), n)
    return out, res


def gemv_f16(w, x, nthreads: int = 0) -> np.ndarray:
    """w [m, k] f16 row-major, x [k] f16 -> f16 [m]."""
    m, k = w.shape
    out = np.zeros(m, dtype=np.float16)
    lib().go_gemv_f16(_u16(w), _u16(x), _u16(out), m, k, nthreads)
    return out


def argmax_f16(logits) -> int:
    return int(lib().go_argmax_f16(_u16(logits), logits.shape[0]))


def silu_mul(gate, up) -> np.ndarray:
    out = np.zeros(gate.shape[0], dtype=np.float16)
    lib().go_silu_mul(_u16(gate), _u16(up), _u16(out), gate.shape[0])
    return out


def qwen3_decode_step(model: dict, token: int, position: int, block_n: int, num_splits: int,
                      fused_ranges: bool = False):
    """One decode token step of src/model.rs:3118-3648, composed of this
    oracle's ops in the graph's order.  `model` holds numpy f16 arrays
    (embed_tokens, final_norm, lm_head, inv_freq (f32), layers: list of dicts
    with input_norm, qkv_proj, q_norm, k_norm, o_proj, post_attn_norm,
    gate_up_proj, down_proj, k_cache, v_cache) and eps, qk_scale_f16_bits,
    num_q_heads, num_kv_heads.  Writes the caches at `position` in place.
    fused_ranges: attention splits on the fused decode step's boundaries.
    Returns (logits f16 [vocab], next token)."""
    hq, hkv, eps = model["num_q_heads"], model["num_kv_heads"], model["eps"]
    D = 128
    G = hq // hkv
    row = model["embed_tokens"][token]                       # :3120-3128
    zero = np.zeros_like(row)
    normed, hidden = add_rms_norm(row, zero, model["layers"][0]["input_norm"], eps)  # :3133-3149
    hidden_after_attn = ff_down = None
    for li, L in enumerate(model["layers"]):
        if li > 0:                                           # :3151-3163
            normed, hidden = add_rms_norm(hidden_after_attn, ff_down, L["input_norm"], eps)
        qkv = gemv_f16(L["qkv_proj"], normed)                # :3170-3176
        q_out = np.zeros(((hq + hkv) * D,), np.float16)
        qk_norm_rope_kv_decode(qkv, L["q_norm"], L["k_norm"], model["inv_freq"], q_out,
                               L["k_cache"], L["v_cache"], position, eps, hq, hkv)
        qg = q_out[:hq * D].reshape(hkv, G, D)
        att, lse = attn_decode_split(qg, L["k_cache"], L["v_cache"], model["qk_scale_f16_bits"],
                                     position, block_n, num_splits, fused_ranges=fused_ranges)
        attn_out = attn_decode_merge(att, lse, G).reshape(-1)
        attn_proj = gemv_f16(L["o_proj"], attn_out)          # :3505-3511
        normed, hidden_after_attn = add_rms_norm(hidden, attn_proj, L["post_attn_norm"], eps)
        gate_up = gemv_f16(L["gate_up_proj"], normed)        # :3529-3535
        inter = gate_up.shape[0] // 2
        ff = silu_mul(gate_up[:inter], gate_up[inter:])      # :3556-3565
        ff_down = gemv_f16(L["down_proj"], ff)               # :3568-3574
    normed, hidden = add_rms_norm(hidden_after_attn, ff_down, model["final_norm"], eps)
    logits = gemv_f16(model["lm_head"], normed)              # :3612-3620
    return logits, argmax_f16(logits)                        # :3622-3640


CAST_DTYPES = {"F16": 0, "BF16": 1, "F32": 2, "F64": 3}


def cast_to_f16(raw: np.ndarray, dtype: str) -> np.ndarray:
    """Raw little-endian element bytes of a safetensors tensor -> f16."""
    if dtype not in CAST_DTYPES:
        raise ValueError(f"unsupported dtype for fp16 cast: {dtype}")
    raw = np.ascontiguousarray(raw).view(np.uint8)
    width = {"F16": 2, "BF16": 2, "F32": 4, "F64": 8}[dtype]
    n = raw.size // width
    out = np.zeros(n, dtype=np.float16)
    st = lib().go_cast_to_f16(raw.ctypes.data_as(ctypes.c_void_p), CAST_DTYPES[dtype], _u16(out), n)
    if st != 0:
        raise ValueError(f"unsupported dtype {dtype}")
    return out
