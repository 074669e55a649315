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
