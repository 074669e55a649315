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
