"""Shared input generators and comparison helpers for the parity tests."""
from __future__ import annotations

import numpy as np

D = 128
EPS = 1e-6
THETA = 1e6
SEED_BASE = 0x67726F7574000000  # "grout\0\0\0"; config c uses SEED_BASE + c

# North-star tolerance for attention outputs against the fp32 oracle.
ATOL = 2e-3
RTOL = 1e-2


def rng(seed_offset: int) -> np.random.Generator:
    return np.random.default_rng(SEED_BASE + seed_offset)


def normal_f16(g: np.random.Generator, shape, scale: float = 1.0) -> np.ndarray:
    return (g.standard_normal(shape, dtype=np.float32) * np.float32(scale)).astype(np.float16)


def norm_weight(g: np.random.Generator) -> np.ndarray:
    """Per-head RMSNorm weight 1 + N(0, 0.1), f16."""
    return (1.0 + 0.1 * g.standard_normal(D, dtype=np.float32)).astype(np.float16)


def f16_ulp_diff(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """|a - b| in units of the f16 grid (ordered bit distance, sign-aware)."""
    ai = a.astype(np.float16).view(np.int16).astype(np.int32)
    bi = b.astype(np.float16).view(np.int16).astype(np.int32)
    ai = np.where(ai < 0, -32768 - ai, ai)
    bi = np.where(bi < 0, -32768 - bi, bi)
    return np.abs(ai - bi)


def assert_close_attn(actual: np.ndarray, expected: np.ndarray, what: str,
                      atol: float = ATOL, rtol: float = RTOL):
    a = actual.astype(np.float32)
    e = expected.astype(np.float32)
    assert np.all(np.isfinite(a)), f"{what}: non-finite output"
    err = np.abs(a - e)
    bad = err > atol + rtol * np.abs(e)
    if bad.any():
        i = np.unravel_index(np.argmax(err - rtol * np.abs(e)), err.shape)
        raise AssertionError(
            f"{what}: {int(bad.sum())} of {bad.size} outside |a-b| <= {atol} + {rtol}|b|; "
            f"worst at {i}: actual {a[i]}, expected {e[i]}, max_abs {err.max():.3e}")
    return float(err.max())


def qk_scale_f16_bits() -> int:
    """f16::from_f32(1/sqrt(128)) (src/model.rs:3427) = 0x2da8."""
    return int(np.float16(np.float32(1.0) / np.sqrt(np.float32(D))).view(np.uint16))


def f16_bits_to_f32(bits: int) -> float:
    return float(np.array([bits], dtype=np.uint16).view(np.float16)[0])


def qwen3_tiny_model(seed_offset: int, layers: int = 2, hidden: int = 256, hq: int = 4,
                     hkv: int = 2, inter: int = 512, vocab: int = 1000, max_seq: int = 64,
                     filled: int = 20, logit_scale: float = 4.0) -> dict:
    """A small random Qwen3-shaped decode model (numpy, f16): weights scaled
    so activations stay O(1), KV caches holding N(0,1) rows at positions
    [0, filled) and zeros after."""
    g = rng(seed_offset)

    def lin(m, k, scale=1.0):
        return normal_f16(g, (m, k), scale / np.sqrt(k))

    def nw(n):
        return (1.0 + 0.1 * g.standard_normal(n, dtype=np.float32)).astype(np.float16)

    def cache():
        c = np.zeros((hkv, max_seq, D), np.float16)
        c[:, :filled] = normal_f16(g, (hkv, filled, D))
        return c

    m = {"num_q_heads": hq, "num_kv_heads": hkv, "eps": EPS,
         "qk_scale_f16_bits": qk_scale_f16_bits(), "layers": []}
    for _ in range(layers):
        m["layers"].append({
            "input_norm": nw(hidden), "qkv_proj": lin((hq + 2 * hkv) * D, hidden),
            "q_norm": nw(D), "k_norm": nw(D), "o_proj": lin(hidden, hq * D),
            "post_attn_norm": nw(hidden), "gate_up_proj": lin(2 * inter, hidden),
            "down_proj": lin(hidden, inter), "k_cache": cache(), "v_cache": cache()})
    m["embed_tokens"] = normal_f16(g, (vocab, hidden))
    m["final_norm"] = nw(hidden)
    m["lm_head"] = lin(vocab, hidden, logit_scale)
    import oracle

    m["inv_freq"] = oracle.build_inv_freq(THETA)
    return m


def write_qwen3_checkpoint(path: str, seed_offset: int, layers: int = 2, hidden: int = 256,
                           hq: int = 4, hkv: int = 2, inter: int = 512, vocab: int = 1000,
                           tie: bool = False) -> dict:
    """A Hugging Face-layout Qwen3 checkpoint in `path`: config.json,
    model.safetensors.index.json and two shards, matrices stored as BF16, the
    embedding as F16, norms as F32 and the q/k norms of layer 0 as F64 (every
    dtype the loader converts).  Returns {name: (dtype, torch tensor)}."""
    import json
    import os

    import torch
    from safetensors.torch import save_file

    g = torch.Generator().manual_seed(SEED_BASE % (1 << 62) + seed_offset)

    def rnd(*shape, scale=1.0):
        return torch.randn(shape, generator=g) * scale

    tensors = {"model.embed_tokens.weight": rnd(vocab, hidden).half(),
               "model.norm.weight": (1 + 0.1 * rnd(hidden)).float()}
    if not tie:
        tensors["lm_head.weight"] = rnd(vocab, hidden, scale=4 / hidden ** 0.5).bfloat16()
    for i in range(layers):
        p = f"model.layers.{i}."
        nd = torch.float64 if i == 0 else torch.float32
        tensors.update({
            p + "input_layernorm.weight": (1 + 0.1 * rnd(hidden)).float(),
            p + "post_attention_layernorm.weight": (1 + 0.1 * rnd(hidden)).float(),
            p + "self_attn.q_proj.weight": rnd(hq * D, hidden, scale=hidden ** -0.5).bfloat16(),
            p + "self_attn.k_proj.weight": rnd(hkv * D, hidden, scale=hidden ** -0.5).bfloat16(),
            p + "self_attn.v_proj.weight": rnd(hkv * D, hidden, scale=hidden ** -0.5).bfloat16(),
            p + "self_attn.o_proj.weight": rnd(hidden, hq * D, scale=(hq * D) ** -0.5).bfloat16(),
            p + "self_attn.q_norm.weight": (1 + 0.1 * rnd(D)).to(nd),
            p + "self_attn.k_norm.weight": (1 + 0.1 * rnd(D)).to(nd),
            p + "mlp.gate_proj.weight": rnd(inter, hidden, scale=hidden ** -0.5).bfloat16(),
            p + "mlp.up_proj.weight": rnd(inter, hidden, scale=hidden ** -0.5).bfloat16(),
            p + "mlp.down_proj.weight": rnd(hidden, inter, scale=inter ** -0.5).bfloat16(),
        })
    names = sorted(tensors)
    shards = {"model-00001-of-00002.safetensors": names[: len(names) // 2],
              "model-00002-of-00002.safetensors": names[len(names) // 2:]}
    weight_map = {}
    for shard, ns in shards.items():
        save_file({n: tensors[n].contiguous() for n in ns}, os.path.join(path, shard),
                  metadata={"format": "pt"})
        weight_map.update({n: shard for n in ns})
    with open(os.path.join(path, "model.safetensors.index.json"), "w") as fh:
        json.dump({"metadata": {"total_size": 0}, "weight_map": weight_map}, fh)
    cfg = {"architectures": ["Qwen3ForCausalLM"], "vocab_size": vocab, "hidden_size": hidden,
           "intermediate_size": inter, "num_hidden_layers": layers, "num_attention_heads": hq,
           "num_key_value_heads": hkv, "head_dim": D, "rms_norm_eps": EPS, "rope_theta": THETA,
           "max_position_embeddings": 40960, "tie_word_embeddings": tie,
           "use_sliding_window": False, "eos_token_id": 151645, "torch_dtype": "bfloat16"}
    with open(os.path.join(path, "config.json"), "w") as fh:
        json.dump(cfg, fh)
    st = {torch.float16: "F16", torch.bfloat16: "BF16", torch.float32: "F32",
          torch.float64: "F64"}
    return {n: (st[t.dtype], t) for n, t in tensors.items()}


def raw_bytes(t) -> np.ndarray:
    """The little-endian element bytes of a CPU torch tensor, as stored by safetensors."""
    import torch

    width = t.element_size()
    return t.contiguous().view(torch.uint8 if width == 1 else
                               {2: torch.int16, 4: torch.int32, 8: torch.int64}[width]
                               ).numpy().view(np.uint8).reshape(-1)
