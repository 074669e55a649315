"""grout_amd — MI355X-native Qwen3 attention hot path of NikVisel/grout.

The product is the C-ABI library ``libgrout_attn_hip.so`` (hand-written HIP for
gfx950, declared in ``include/grout_attn_hip.h``).  This package is the host-side
mirror of grout's operator interface for that path, the same names, argument
meaning and error behaviour as the Rust call sites it replaces:

=====================================  ==========================================
grout (Rust, src/)                     here
=====================================  ==========================================
build_inv_freq (model.rs:5992)         :func:`build_inv_freq`
execute_qk_norm_rope_kv_prefill_op_ctx :func:`qk_norm_rope_kv_prefill`
  (model.rs:4463)
qk_norm_rope_kv_decode_raw_f16 record  :func:`qk_norm_rope_kv_decode`
  (model.rs:3194)
attend_seq_arc_into_ctx_with_position  :func:`attend_prefill`
  (model.rs:5556), Host position
fmha_decode_gqa_split record           :func:`fmha_decode_gqa_split`
  (model.rs:3428)
splitk_reduce_merge record             :func:`splitk_reduce_merge`
  (model.rs:3453)
DecodeCudaGraphRunner (model.rs:318)   :class:`DecodeGraphRunner`
=====================================  ==========================================

Tensors are torch tensors on the GPU (PyTorch is plumbing for device memory and
streams here); every op launches on ``torch.cuda.current_stream()``.  Shape
checks raise :class:`GroutError` with the reference's ``ensure!`` message before
anything is launched; a non-zero status from the library also raises.
"""
from __future__ import annotations

import ctypes
import math

from . import _lib
from ._lib import GROUT_OK, LibraryMissing

__all__ = [
    "GroutError", "LibraryMissing", "lib", "build_inv_freq", "qk_norm_rope_kv_prefill",
    "qk_norm_rope_kv_decode", "attend_prefill", "fmha_decode_gqa_split",
    "splitk_reduce_merge", "decode_fused", "attend_prefill_split", "prefill_split_scratch",
    "prefill_splitk_reduce_merge", "add_rms_norm_decode", "gemv_f16", "gemv_silu_mul", "argmax_scratch",
    "argmax_f16", "embed_rms_norm_decode", "silu_mul", "Qwen3DecodeRunner", "QWEN3_LAYER_KEYS",
    "decode_scratch", "decode_counters",
    "pick_num_splits", "DecodeGraphRunner",
    "HEAD_DIM", "ATTN_BN_DECODE",
]

HEAD_DIM = 128
# src/model.rs:128 ATTN_BN_DECODE: KV tile of the decode split boundaries.
ATTN_BN_DECODE = 32


class GroutError(RuntimeError):
    """A rejected argument (reference ``ensure!``) or a failed launch."""

    def __init__(self, message: str, status: int | None = None):
        super().__init__(message)
        self.status = status


def lib():
    return _lib.load()


def _check(status: int, what: str):
    if status != GROUT_OK:
        text = lib().grout_status_string(status).decode()
        name = _lib.STATUS_NAMES.get(status, f"hipError {status}")
        raise GroutError(f"{what}: {name} ({text})", status)


def _ensure(cond: bool, msg: str):
    if not cond:
        raise GroutError(msg)


def _torch():
    import torch
    return torch


def _ptr(t) -> int:
    return t.data_ptr()


def _stream() -> int:
    torch = _torch()
    return torch.cuda.current_stream().cuda_stream


def _f16(t, name: str):
    torch = _torch()
    _ensure(t.dtype == torch.float16, f"{name} must be f16, got {t.dtype}")
    _ensure(t.is_cuda, f"{name} must be a device tensor")
    _ensure(t.is_contiguous(), f"{name} must be contiguous")


def build_inv_freq(theta: float, head_dim: int = HEAD_DIM):
    """src/model.rs:5992-6003 on the host (f32); returns a CPU float32 tensor."""
    torch = _torch()
    out = (ctypes.c_float * (head_dim // 2))()
    _check(lib().grout_build_inv_freq(float(theta), head_dim, out), "build_inv_freq")
    return torch.tensor(list(out), dtype=torch.float32)


def qk_norm_rope_kv_prefill(q, k, v, q_weight, k_weight, inv_freq, out, k_cache, v_cache,
                            eps: float, position_start: int):
    """execute_qk_norm_rope_kv_prefill_op_ctx (src/model.rs:4463-4598).

    q [S,Hq,D], k/v [S,Hkv,D], out [S,Hq,D]; writes cache rows
    [position_start, position_start+S) of k_cache/v_cache [Hkv,MS,D]."""
    _ensure(q.dim() == 3, f"q shape mismatch in fused qk/rope/kv prefill: {list(q.shape)}")
    S, Hq, D = q.shape
    _ensure(k.dim() == 3 and k.shape[0] == S and k.shape[2] == D,
            f"k shape mismatch in fused qk/rope/kv prefill: {list(k.shape)}")
    Hkv = k.shape[1]
    _ensure(list(v.shape) == [S, Hkv, D],
            f"v shape mismatch in fused qk/rope/kv prefill: {list(v.shape)}")
    _ensure(list(out.shape) == [S, Hq, D],
            f"fused qk/rope/kv output shape mismatch: {list(out.shape)}")
    _ensure(D % 2 == 0, f"fused qk/rope/kv requires even head_dim, got {D}")
    MS = k_cache.shape[1] if k_cache.dim() == 3 else -1
    _ensure(position_start + S <= MS,
            f"fused qk/rope/kv range [{position_start}..{position_start + S}) exceeds "
            f"max_seq_len {MS}")
    _ensure(list(k_cache.shape) == [Hkv, MS, D],
            f"k_cache shape mismatch in fused qk/rope/kv: {list(k_cache.shape)}")
    _ensure(list(v_cache.shape) == [Hkv, MS, D],
            f"v_cache shape mismatch in fused qk/rope/kv: {list(v_cache.shape)}")
    for t, n in ((q, "q"), (k, "k"), (v, "v"), (q_weight, "q_weight"), (k_weight, "k_weight"),
                 (out, "out"), (k_cache, "k_cache"), (v_cache, "v_cache")):
        _f16(t, n)
    _check(lib().grout_qk_norm_rope_kv_prefill(
        _ptr(q), _ptr(k), _ptr(v), _ptr(q_weight), _ptr(k_weight), _ptr(inv_freq), _ptr(out),
        _ptr(k_cache), _ptr(v_cache), float(eps), int(position_start), S, Hq, Hkv, D, MS,
        _stream()), "qk_norm_rope_kv_prefill")
    return out


def _kv_update_checks(new_k, new_v, k_cache, v_cache):
    """The shape ensure!s of kv_cache_update_seq_arc_ctx_with_position
    (src/model.rs:5396-5423); returns (S, Hkv, D, MS)."""
    _ensure(new_k.dim() == 3,
            f"new_k must be rank 3 [seqlen, kv_heads, head_dim], got {list(new_k.shape)}")
    S, Hkv, D = new_k.shape
    _ensure(k_cache.dim() == 3 and k_cache.shape[0] == Hkv and k_cache.shape[2] == D,
            f"new_k shape mismatch: {list(new_k.shape)}")
    _ensure(list(new_v.shape) == [S, Hkv, D], f"new_v shape mismatch: {list(new_v.shape)}")
    MS = k_cache.shape[1]
    _ensure(list(v_cache.shape) == [Hkv, MS, D],
            f"v_cache shape mismatch: {list(v_cache.shape)}")
    for t, n in ((new_k, "new_k"), (new_v, "new_v"), (k_cache, "k_cache"), (v_cache, "v_cache")):
        _f16(t, n)
    return S, Hkv, D, MS


def kv_cache_update_seq(new_k, new_v, k_cache, v_cache, position_start: int):
    """kv_cache_update_seq_arc_ctx_with_position with a host position
    (src/model.rs:5388-5480, kv_cache_update_seq_f16): cache rows
    [position_start, position_start+S) of every KV head take new_k/new_v."""
    S, Hkv, D, MS = _kv_update_checks(new_k, new_v, k_cache, v_cache)
    _ensure(position_start + S <= MS,
            f"kv_cache_update range [{position_start}..{position_start + S}) exceeds "
            f"max_seq_len {MS}")
    _check(lib().grout_kv_cache_update_seq(
        _ptr(new_k), _ptr(new_v), _ptr(k_cache), _ptr(v_cache), int(position_start), S, Hkv, D,
        MS, _stream()), "kv_cache_update_seq")


def kv_cache_update_seq_dynpos(new_k, new_v, k_cache, v_cache, position):
    """The device-position form (src/model.rs:5433-5441, 5483-5502,
    kv_cache_update_seq_dynpos_f16): ``position`` is a device u32 tensor of
    shape [1]; the decode-graph path writes one row."""
    S, Hkv, D, MS = _kv_update_checks(new_k, new_v, k_cache, v_cache)
    _ensure(S == 1, f"decode graph path expects seq_len=1, got {S}")
    _ensure(list(position.shape) == [1],
            f"kv_cache position tensor must be shape [1], got {list(position.shape)}")
    _check(lib().grout_kv_cache_update_seq_dynpos(
        _ptr(new_k), _ptr(new_v), _ptr(k_cache), _ptr(v_cache), _ptr(position), S, Hkv, D, MS,
        _stream()), "kv_cache_update_seq_dynpos")


def qk_norm_rope_kv_decode(qkv, q_weight, k_weight, inv_freq, q_out, k_cache, v_cache,
                           position, eps: float, num_q_heads: int, num_kv_heads: int):
    """qk_norm_rope_kv_decode_raw_f16 as recorded at src/model.rs:3194-3221.

    ``position`` is a device u32 tensor of shape [1] (torch.int32 storage)."""
    D = q_weight.shape[0]
    _ensure(qkv.numel() == (num_q_heads + 2 * num_kv_heads) * D,
            f"qkv has {qkv.numel()} elements, expected {(num_q_heads + 2 * num_kv_heads) * D}")
    _ensure(q_out.numel() >= num_q_heads * D, "q_out too small")
    _ensure(position.numel() == 1,
            f"attention position tensor must be shape [1], got {list(position.shape)}")
    MS = k_cache.shape[1]
    _check(lib().grout_qk_norm_rope_kv_decode(
        _ptr(qkv), _ptr(q_weight), _ptr(k_weight), _ptr(inv_freq), _ptr(q_out), _ptr(k_cache),
        _ptr(v_cache), _ptr(position), float(eps), num_q_heads, num_kv_heads, D, MS,
        _stream()), "qk_norm_rope_kv_decode")


def attend_prefill(q, k_cache, v_cache, out, position_start: int,
                   qk_scale: float | None = None, kv_len: int | None = None,
                   sched_counters=None):
    """attend_seq_arc_into_ctx_with_position with a host position (src/model.rs:5556-5834).

    kv_len defaults to position_start + q_len (:5638); qk_scale to 1/sqrt(D) in
    f32 (:5601).  With `sched_counters` (prefill_sched_counters()) the launch
    uses the dynamic per-XCD schedule (grout_attn_prefill_sched); the result
    is bit-identical to the static grid's."""
    _ensure(q.dim() == 3, f"q must be rank 3 [seqlen, heads, head_dim], got {list(q.shape)}")
    q_len, Hq, D = q.shape
    Hkv, MS, _ = k_cache.shape
    _ensure(list(out.shape) == [q_len, Hq, D],
            f"attend output shape mismatch, got {list(out.shape)}")
    if qk_scale is None:
        qk_scale = 1.0 / math.sqrt(float(D))
    if kv_len is None:
        kv_len = position_start + q_len
    for t, n in ((q, "q"), (k_cache, "k_cache"), (v_cache, "v_cache"), (out, "out")):
        _f16(t, n)
    args = (_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(out), float(qk_scale), Hq, Hkv, D, q_len,
            int(kv_len), int(position_start), MS)
    if sched_counters is None:
        _check(lib().grout_attn_prefill(*args, _stream()), "attn_prefill")
    else:
        _ensure(sched_counters.is_cuda and sched_counters.is_contiguous(),
                "sched_counters must be a contiguous device tensor")
        _ensure(sched_counters.numel() * sched_counters.element_size()
                >= lib().grout_attn_prefill_sched_counter_bytes(),
                "sched_counters is smaller than grout_attn_prefill_sched_counter_bytes()")
        _check(lib().grout_attn_prefill_sched(*args, _ptr(sched_counters), _stream()),
               "attn_prefill_sched")
    return out


def prefill_sched_counters(device="cuda"):
    """Zeroed counters for attend_prefill(..., sched_counters=...): every launch
    leaves them zero again.  Launches that overlap on one buffer race."""
    torch = _torch()
    n = lib().grout_attn_prefill_sched_counter_bytes() // 4
    return torch.zeros((n,), dtype=torch.int32, device=device)


def prefill_split_scratch(num_q_heads: int, q_len: int, block_m: int, group: int,
                          num_splits: int, head_dim: int = HEAD_DIM, device="cuda"):
    """Scratch of fmha_prefill_gqa_lpt_split (src/kernels.rs:1922-1944):
    att [tiles, NKS*BM*group, D] f16, lse [tiles, NKS*BM*group] f32 with
    tiles = ceil(q_len/BM) * (Hq/group)."""
    torch = _torch()
    rows = lib().grout_attn_prefill_split_lse_bytes(num_q_heads, q_len, block_m, group,
                                                    num_splits)
    _ensure(rows >= 0, "invalid split-K prefill geometry")
    rows //= 4
    ns_m = num_splits * block_m * group
    att = torch.zeros((rows // ns_m, ns_m, head_dim), dtype=torch.float16, device=device)
    lse = torch.zeros((rows // ns_m, ns_m), dtype=torch.float32, device=device)
    return att, lse


def attend_prefill_split(q, k_cache, v_cache, att_partial, lse_partial, position_start: int,
                         block_m: int, block_n: int, group: int, num_splits: int,
                         qk_scale: float | None = None, kv_len: int | None = None):
    """fmha_prefill_gqa_lpt_split (src/kernels.rs:1872-2142) as the attention
    microbench launches it (benchmarks/src/bin/attention_microbench.rs:411-469),
    on grout's cache layout; writes the normalised per-split partials and LSEs."""
    _ensure(q.dim() == 3, f"q must be rank 3 [seqlen, heads, head_dim], got {list(q.shape)}")
    q_len, Hq, D = q.shape
    Hkv, MS, _ = k_cache.shape
    qgs = Hq // Hkv if Hkv else 0
    _ensure(group >= 1 and qgs % group == 0, f"group must divide q_group_size={qgs}")
    if qk_scale is None:
        qk_scale = 1.0 / math.sqrt(float(D))
    if kv_len is None:
        kv_len = position_start + q_len
    ns_m = num_splits * block_m * group
    tiles = -(-q_len // block_m) * (Hq // group)
    _ensure(list(att_partial.shape) == [tiles, ns_m, D],
            f"att_partial shape mismatch, got {list(att_partial.shape)}")
    _ensure(list(lse_partial.shape) == [tiles, ns_m],
            f"lse_partial shape mismatch, got {list(lse_partial.shape)}")
    for t, n in ((q, "q"), (k_cache, "k_cache"), (v_cache, "v_cache"),
                 (att_partial, "att_partial")):
        _f16(t, n)
    _check(lib().grout_attn_prefill_split(
        _ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(att_partial), _ptr(lse_partial),
        float(qk_scale), Hq, Hkv, D, q_len, int(kv_len), int(position_start), MS, block_m,
        block_n, group, num_splits, _stream()), "fmha_prefill_gqa_lpt_split")


def prefill_splitk_reduce_merge(att_partial, lse_partial, out, block_m: int, group: int,
                                num_splits: int):
    """prefill_splitk_reduce_merge (src/kernels.rs:2151-2323); out [q_len, Hq, D]."""
    q_len, Hq, D = out.shape
    _f16(out, "out")
    _check(lib().grout_attn_prefill_split_merge(
        _ptr(att_partial), _ptr(lse_partial), _ptr(out), Hq, D, q_len, block_m, group,
        num_splits, _stream()), "prefill_splitk_reduce_merge")
    return out


def add_rms_norm_decode(residual, x, weight, out, residual_out, eps: float):
    """add_rms_norm_decode_raw_f16 (src/kernels.rs:3076-3216) on one hidden row:
    residual_out = residual + x, out = RMSNorm(residual_out) * weight."""
    n = residual.numel()
    args = ((residual, "residual"), (x, "x"), (weight, "weight"), (out, "out"),
            (residual_out, "residual_out"))
    for t, nm in args:
        _ensure(t.numel() == n, f"{nm} must have {n} elements, got {t.numel()}")
    for t, nm in args:
        _f16(t, nm)
    _check(lib().grout_add_rms_norm_decode(_ptr(residual), _ptr(x), _ptr(weight), _ptr(out),
                                           _ptr(residual_out), float(eps), n, _stream()),
           "add_rms_norm_decode")
    return out, residual_out


def gemv_f16(weight, x, out):
    """cuBLAS GemvInPlace (src/cublas.rs:572-607): out[m] = weight[m, k] @ x[k], f32 accumulate."""
    _ensure(weight.dim() == 2, f"weight must be [m, k], got {list(weight.shape)}")
    m, k = weight.shape
    _ensure(x.numel() == k, f"x must have {k} elements, got {x.numel()}")
    _ensure(out.numel() == m, f"out must have {m} elements, got {out.numel()}")
    for t, nm in ((weight, "weight"), (x, "x"), (out, "out")):
        _f16(t, nm)
    _check(lib().grout_gemv_f16(_ptr(weight), _ptr(x), _ptr(out), m, k, _stream()), "gemv_f16")
    return out


def gemv_silu_mul(gate_up, x, out):
    """The gate_up GEMV and silu_mul_2d_f16 of the decode graph (src/model.rs:3529-3535,
    3556-3565) in one launch: out[n] = silu(gate) * up of the f16 rows of gate_up[2n, k] @ x,
    bit-identical to gemv_f16 followed by silu_mul."""
    _ensure(gate_up.dim() == 2 and gate_up.shape[0] % 2 == 0,
            f"gate_up must be [2n, k], got {list(gate_up.shape)}")
    m2, k = gate_up.shape
    _ensure(x.numel() == k, f"x must have {k} elements, got {x.numel()}")
    _ensure(out.numel() == m2 // 2, f"out must have {m2 // 2} elements, got {out.numel()}")
    for t, nm in ((gate_up, "gate_up"), (x, "x"), (out, "out")):
        _f16(t, nm)
    _check(lib().grout_gemv_silu_mul_f16(_ptr(gate_up), _ptr(x), _ptr(out), m2 // 2, k, _stream()),
           "gemv_silu_mul_f16")
    return out


def argmax_scratch(n: int, device="cuda"):
    """Per-block scratch of :func:`argmax_f16` for n logits."""
    torch = _torch()
    nb = int(lib().grout_argmax_blocks(n))
    _ensure(nb > 0, "argmax needs at least one logit")
    return (torch.empty((nb,), dtype=torch.float32, device=device),
            torch.empty((nb,), dtype=torch.int32, device=device))


def argmax_f16(logits, block_max, block_idx, token):
    """argmax_blocks_f16 + argmax_reduce_blocks_to_u32 (src/kernels.rs:345-505):
    token[0] = lowest index of the largest logit."""
    _f16(logits, "logits")
    _check(lib().grout_argmax_f16(_ptr(logits), _ptr(block_max), _ptr(block_idx), _ptr(token),
                                  logits.numel(), _stream()), "argmax_f16")
    return token


def embed_rms_norm_decode(token, table, weight, out, residual_out, eps: float):
    """embedding_batch_f16 + rms_norm_f16 (src/kernels.rs:693-711, 304-344) for the
    device token id token[0]: residual_out = table[token], out = RMSNorm(row) * weight."""
    _ensure(table.dim() == 2, f"table must be [vocab, n], got {list(table.shape)}")
    vocab, n = table.shape
    for t, nm in ((weight, "weight"), (out, "out"), (residual_out, "residual_out")):
        _ensure(t.numel() == n, f"{nm} must have {n} elements, got {t.numel()}")
    for t, nm in ((table, "table"), (weight, "weight"), (out, "out"),
                  (residual_out, "residual_out")):
        _f16(t, nm)
    _check(lib().grout_embed_rms_norm_decode(_ptr(token), _ptr(table), vocab, _ptr(weight),
                                             _ptr(out), _ptr(residual_out), float(eps), n,
                                             _stream()), "embed_rms_norm_decode")
    return out, residual_out


def silu_mul(gate, up, out):
    """silu_mul_2d_f16 (src/kernels.rs:271-301): out = sigmoid(gate) * gate * up."""
    n = out.numel()
    _ensure(gate.numel() == n and up.numel() == n, "gate, up and out must have equal sizes")
    for t, nm in ((gate, "gate"), (up, "up"), (out, "out")):
        _f16(t, nm)
    _check(lib().grout_silu_mul_f16(_ptr(gate), _ptr(up), _ptr(out), n, _stream()), "silu_mul")
    return out


QWEN3_LAYER_KEYS = ("input_norm", "qkv_proj", "q_norm", "k_norm", "o_proj", "post_attn_norm",
                    "gate_up_proj", "down_proj", "k_cache", "v_cache")


class Qwen3DecodeRunner:
    """DecodeCudaGraphRunner (src/model.rs:318-493) with the graph of
    src/model.rs:3118-3648: the whole Qwen3 decode step (embedding, every
    layer's norms, GEMVs, attention and MLP, final norm, lm_head, greedy
    argmax) captured once into a hipGraph over borrowed weights and caches.

    `layers` holds one dict per layer with the keys of QWEN3_LAYER_KEYS;
    `token` and `position` are device int32[1] tensors (the step reads the
    token and writes the next one in place), `logits` a device f16[vocab]."""

    def __init__(self, *, layers, embed_tokens, final_norm, lm_head, inv_freq, token, position,
                 logits, num_q_heads: int, num_kv_heads: int, eps: float,
                 qk_scale_f16_bits: int, num_splits: int | None = None,
                 block_n: int = ATTN_BN_DECODE, prime_position: int = 0, stream=None):
        torch = _torch()
        _ensure(len(layers) >= 1, "at least one layer")
        _ensure(embed_tokens.dim() == 2, "embed_tokens must be [vocab, hidden]")
        vocab, hidden = embed_tokens.shape
        hq, hkv = num_q_heads, num_kv_heads
        _ensure(hq > 0 and hkv > 0 and hq % hkv == 0,
                f"num_q_heads {hq} must be a multiple of num_kv_heads {hkv}")
        d = HEAD_DIM
        inter = layers[0]["down_proj"].shape[1]
        max_seq = layers[0]["k_cache"].shape[1]
        shapes = {"input_norm": (hidden,), "qkv_proj": ((hq + 2 * hkv) * d, hidden),
                  "q_norm": (d,), "k_norm": (d,), "o_proj": (hidden, hq * d),
                  "post_attn_norm": (hidden,), "gate_up_proj": (2 * inter, hidden),
                  "down_proj": (hidden, inter), "k_cache": (hkv, max_seq, d),
                  "v_cache": (hkv, max_seq, d)}
        # Shapes first (the reference's ensure! order), then dtypes and devices.
        for i, L in enumerate(layers):
            for key in QWEN3_LAYER_KEYS:
                _ensure(key in L, f"layer {i} has no {key}")
                _ensure(tuple(L[key].shape) == shapes[key],
                        f"layer {i} {key} shape {list(L[key].shape)} != {list(shapes[key])}")
        _ensure(tuple(lm_head.shape) == (vocab, hidden), "lm_head must be [vocab, hidden]")
        _ensure(final_norm.numel() == hidden and logits.numel() == vocab,
                "final_norm [hidden] and logits [vocab] expected")
        for i, L in enumerate(layers):
            for key in QWEN3_LAYER_KEYS:
                _f16(L[key], f"layer {i} {key}")
        for t, nm in ((embed_tokens, "embed_tokens"), (lm_head, "lm_head"),
                      (final_norm, "final_norm"), (logits, "logits")):
            _f16(t, nm)
        _ensure(inv_freq.dtype == torch.float32 and inv_freq.is_cuda and inv_freq.numel() == 64,
                "inv_freq must be a device float32 [64] tensor (build_inv_freq)")
        for t, nm in ((token, "token"), (position, "position")):
            _ensure(t.dtype in (torch.int32, torch.uint32) and t.is_cuda and t.numel() >= 1,
                    f"{nm} must be a device int32 tensor")
        if num_splits is None:
            num_splits = pick_num_splits(max_seq, hkv, block_n, group=hq // hkv)
        self._layers = (_lib.Qwen3Layer * len(layers))(*[
            _lib.Qwen3Layer(**{key: _ptr(L[key]) for key in QWEN3_LAYER_KEYS}) for L in layers])
        M = _lib.Qwen3Model(
            num_layers=len(layers), hidden=hidden, intermediate=inter, vocab=vocab,
            num_q_heads=hq, num_kv_heads=hkv, head_dim=d, max_seq_len=max_seq, block_n=block_n,
            num_splits=num_splits, eps=float(eps), qk_scale_f16=int(qk_scale_f16_bits),
            layers=self._layers, embed_tokens=_ptr(embed_tokens), final_norm=_ptr(final_norm),
            lm_head=_ptr(lm_head), inv_freq=_ptr(inv_freq), token=_ptr(token),
            d_position=_ptr(position), logits=_ptr(logits), workspace=None)
        nbytes = int(lib().grout_qwen3_workspace_bytes(ctypes.byref(M)))
        _check(nbytes if nbytes < 0 else 0, "qwen3_workspace_bytes")
        self.workspace = torch.empty((nbytes,), dtype=torch.uint8, device=embed_tokens.device)
        M.workspace = self.workspace.data_ptr()
        _ensure(M.workspace % 256 == 0, "workspace must be 256-byte aligned")
        self._model = M
        self.num_splits = num_splits
        self._keep = (layers, embed_tokens, final_norm, lm_head, inv_freq, token, position, logits)
        self.stream = stream if stream is not None else torch.cuda.Stream()
        torch.cuda.current_stream().synchronize()  # caller's buffers are ready
        h = ctypes.c_void_p()
        _check(lib().grout_qwen3_runner_create(ctypes.byref(M), int(prime_position),
                                               self.stream.cuda_stream, ctypes.byref(h)),
               "qwen3_runner_create")
        self._h = h

    def seed_token(self, token: int):
        _check(lib().grout_qwen3_runner_seed_token(self._h, int(token)), "qwen3_seed_token")

    def step(self, position: int) -> int:
        """launch_step: one replay at `position`; returns the token it picked."""
        out = ctypes.c_uint32()
        _check(lib().grout_qwen3_runner_step(self._h, int(position), ctypes.byref(out)),
               "qwen3_runner_step")
        return int(out.value)

    def run(self, first_position: int, count: int):
        """`count` replays from `first_position`, each embedding the previous token.

        Asynchronous on :attr:`stream`: synchronise it (or wait on an event
        recorded on it) before reading logits, the token or the caches."""
        _check(lib().grout_qwen3_runner_run(self._h, int(first_position), int(count)),
               "qwen3_runner_run")

    def eager_step(self):
        """The same step launched op by op on the runner's stream (no graph)."""
        _check(lib().grout_qwen3_decode_step(ctypes.byref(self._model), self.stream.cuda_stream),
               "qwen3_decode_step")

    def close(self):
        if getattr(self, "_h", None):
            _check(lib().grout_qwen3_runner_destroy(self._h), "qwen3_runner_destroy")
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def pick_num_splits(max_context: int, num_kv_heads: int, block_n: int = ATTN_BN_DECODE,
                    device: int | None = None, group: int = 1) -> int:
    """Split count of the decode graph for this device's CU count
    (grout_attn_decode_pick_splits_grouped; group = query heads per KV head)."""
    torch = _torch()
    cu = ctypes.c_int32(0)
    dev = torch.cuda.current_device() if device is None else device
    _check(lib().grout_device_cu_count(dev, ctypes.byref(cu)), "device_cu_count")
    return int(lib().grout_attn_decode_pick_splits_grouped(cu.value, num_kv_heads, group,
                                                           max_context, block_n))


def decode_scratch(num_kv_heads: int, group: int, num_splits: int, head_dim: int = HEAD_DIM,
                   device="cuda"):
    """Split-K scratch (src/model.rs:2508-2525): att [Hkv, NKS*G, D] f16, lse [Hkv, NKS*G] f32."""
    torch = _torch()
    att = torch.zeros((num_kv_heads, num_splits * group, head_dim), dtype=torch.float16,
                      device=device)
    lse = torch.zeros((num_kv_heads, num_splits * group), dtype=torch.float32, device=device)
    return att, lse


def decode_counters(num_kv_heads: int, device="cuda"):
    """Zeroed merge counters for :func:`decode_fused`
    (grout_attn_decode_counter_bytes bytes, int32 storage)."""
    torch = _torch()
    nbytes = int(lib().grout_attn_decode_counter_bytes(num_kv_heads))
    return torch.zeros((nbytes // 4,), dtype=torch.int32, device=device)


def decode_fused(qkv, q_weight, k_weight, inv_freq, q_out, k_cache, v_cache, att_partial,
                 lse_partial, out, counters, position, eps: float, qk_scale_f16_bits: int,
                 num_q_heads: int, num_kv_heads: int, block_n: int = ATTN_BN_DECODE,
                 advance_position: bool = False):
    """One decode step in one launch: the QK norm/RoPE/KV write, split-K GQA
    attention and merge that grout records as three ops (src/model.rs:3194-3221,
    3428-3473).  Writes q_out rows [0, Hq), the cache row at *position and out
    [Hkv, G, D]; with advance_position the device position ends one higher."""
    D = q_weight.shape[0]
    G = num_q_heads // num_kv_heads
    _ensure(qkv.numel() == (num_q_heads + 2 * num_kv_heads) * D, "qkv size mismatch")
    _ensure(att_partial.dim() == 3 and att_partial.shape[1] % G == 0, "att_partial shape mismatch")
    ns = att_partial.shape[1] // G
    _ensure(counters.numel() * 4 >= lib().grout_attn_decode_counter_bytes(num_kv_heads),
            "counters too small")
    _check(lib().grout_attn_decode_fused(
        _ptr(qkv), _ptr(q_weight), _ptr(k_weight), _ptr(inv_freq), _ptr(q_out), _ptr(k_cache),
        _ptr(v_cache), _ptr(att_partial), _ptr(lse_partial), _ptr(out), _ptr(counters),
        _ptr(position), float(eps), int(qk_scale_f16_bits), num_q_heads, num_kv_heads, D,
        k_cache.shape[1], block_n, ns, 1 if advance_position else 0, _stream()),
        "decode_fused")
    return out


def fmha_decode_gqa_split(q_grouped, k_cache, v_cache, att_partial, lse_partial,
                          qk_scale_f16_bits: int, position, block_n: int = ATTN_BN_DECODE):
    """fmha_decode_gqa_split as recorded at src/model.rs:3428-3452; q_grouped [Hkv, G, D]."""
    Hkv, G, D = q_grouped.shape
    _ensure(att_partial.dim() == 3 and att_partial.shape[0] == Hkv
            and att_partial.shape[1] % G == 0, "att_partial shape mismatch")
    ns = att_partial.shape[1] // G
    _ensure(list(lse_partial.shape) == [Hkv, ns * G], "lse_partial shape mismatch")
    _check(lib().grout_attn_decode_split(
        _ptr(q_grouped), _ptr(k_cache), _ptr(v_cache), _ptr(att_partial), _ptr(lse_partial),
        int(qk_scale_f16_bits), _ptr(position), Hkv, G, D, k_cache.shape[1], block_n, ns,
        _stream()), "fmha_decode_gqa_split")


def splitk_reduce_merge(att_partial, lse_partial, out):
    """splitk_reduce_merge as recorded at src/model.rs:3453-3473; out [Hkv, G, D]."""
    Hkv, G, D = out.shape
    ns = att_partial.shape[1] // G
    _check(lib().grout_attn_decode_merge(
        _ptr(att_partial), _ptr(lse_partial), _ptr(out), Hkv, G, D, ns, _stream()),
        "splitk_reduce_merge")
    return out


class DecodeGraphRunner:
    """Attention slice of DecodeCudaGraphRunner (src/model.rs:318-493).

    Captures the fused decode step (norm/RoPE/KV write, split-K decode, merge)
    for one layer's buffers into a hipGraph; :meth:`launch_step` writes the
    device position and replays it (no host sync); :meth:`run` writes it once
    and lets each replay advance it."""

    def __init__(self, *, qkv, q_weight, k_weight, inv_freq, q_out, k_cache, v_cache,
                 att_partial, lse_partial, attn_out, position, eps: float,
                 qk_scale_f16_bits: int, num_q_heads: int, num_kv_heads: int,
                 num_splits: int, block_n: int = ATTN_BN_DECODE, prime_position: int = 0,
                 counters=None, stream=None):
        torch = _torch()
        if counters is None:
            counters = decode_counters(num_kv_heads, device=k_cache.device)
        self.counters = counters
        self._keep = (qkv, q_weight, k_weight, inv_freq, q_out, k_cache, v_cache, att_partial,
                      lse_partial, attn_out, position, counters)
        self.stream = stream if stream is not None else torch.cuda.Stream()
        torch.cuda.current_stream().synchronize()  # caller's buffers are ready
        L = _lib.DecodeLayer(
            qkv=_ptr(qkv), q_weight=_ptr(q_weight), k_weight=_ptr(k_weight),
            inv_freq=_ptr(inv_freq), q_out=_ptr(q_out), k_cache=_ptr(k_cache),
            v_cache=_ptr(v_cache), att_partial=_ptr(att_partial),
            lse_partial=_ptr(lse_partial), attn_out=_ptr(attn_out),
            d_position=_ptr(position), counters=_ptr(counters), eps=float(eps),
            qk_scale_f16=int(qk_scale_f16_bits),
            num_q_heads=num_q_heads, num_kv_heads=num_kv_heads, head_dim=q_weight.shape[0],
            max_seq_len=k_cache.shape[1], block_n=block_n, num_splits=num_splits)
        self._layer = L
        h = ctypes.c_void_p()
        _check(lib().grout_decode_runner_create(ctypes.byref(L), int(prime_position),
                                                self.stream.cuda_stream, ctypes.byref(h)),
               "decode_runner_create")
        self._h = h

    def launch_step(self, position: int):
        """Writes the device position, then replays the graph, both on
        :attr:`stream`; synchronise it before reading attn_out or the caches."""
        _check(lib().grout_decode_runner_step(self._h, int(position)), "decode_runner_step")

    def run(self, first_position: int, count: int):
        """`count` consecutive steps from `first_position`, issued from C without
        returning to Python between steps (the graph advances the position).
        Asynchronous on :attr:`stream`, as :meth:`launch_step`."""
        _check(lib().grout_decode_runner_run(self._h, int(first_position), int(count)),
               "decode_runner_run")

    def zero_kv_caches(self):
        _check(lib().grout_decode_runner_zero_kv(self._h), "decode_runner_zero_kv")

    def close(self):
        if getattr(self, "_h", None):
            _check(lib().grout_decode_runner_destroy(self._h), "decode_runner_destroy")
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
