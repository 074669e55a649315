"""GPU parity of the fused QK RMSNorm + RoPE + KV write against the oracle.

Contract: KV slot indexing bit-exact, V copied bit-exactly, Q/K within 1 f16
ulp of the f32 restatement of src/kernels.rs:3415-4016.
"""
import numpy as np
import pytest

import oracle
from tests._util import D, EPS, THETA, f16_ulp_diff, norm_weight, normal_f16, rng

pytestmark = pytest.mark.gpu


def _to_dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def _run_prefill(torch, q, k, v, qw, kw, inv, k_cache, v_cache, ps):
    import grout_amd

    dq, dk, dv = _to_dev(torch, q), _to_dev(torch, k), _to_dev(torch, v)
    dqw, dkw = _to_dev(torch, qw), _to_dev(torch, kw)
    dinv = _to_dev(torch, inv)
    dkc, dvc = _to_dev(torch, k_cache), _to_dev(torch, v_cache)
    dout = torch.zeros_like(dq)
    grout_amd.qk_norm_rope_kv_prefill(dq, dk, dv, dqw, dkw, dinv, dout, dkc, dvc, EPS, ps)
    torch.cuda.synchronize()
    return dout.cpu().numpy(), dkc.cpu().numpy(), dvc.cpu().numpy()


@pytest.mark.parametrize("hq,hkv,S,ps,MS,seed", [
    (16, 8, 512, 0, 512, 1),        # config c1 (Qwen3-0.6B layer)
    (32, 8, 300, 17, 400, 2),       # ragged S, nonzero position_start
    (4, 2, 1, 0, 16, 3),            # single token
    (64, 8, 70, 32700, 32770, 4),   # Qwen3-32B heads, positions near 32K (large RoPE angles)
    (32, 8, 4096, 0, 4096, 5),      # multi-token workgroups (4096 rows per launch)
])
def test_prefill_matches_oracle(gpu, hq, hkv, S, ps, MS, seed):
    import torch

    g = rng(seed)
    q, k, v = normal_f16(g, (S, hq, D)), normal_f16(g, (S, hkv, D)), normal_f16(g, (S, hkv, D))
    qw, kw = norm_weight(g), norm_weight(g)
    inv = oracle.build_inv_freq(THETA)
    # Sentinel-filled caches: every slot outside [ps, ps+S) must stay untouched.
    sentinel = np.float16(-7.25)
    kc0 = np.full((hkv, MS, D), sentinel, dtype=np.float16)
    vc0 = np.full((hkv, MS, D), sentinel, dtype=np.float16)

    out, kc, vc = _run_prefill(torch, q, k, v, qw, kw, inv, kc0, vc0, ps)

    kc_ref, vc_ref = kc0.copy(), vc0.copy()
    q_ref = oracle.qk_norm_rope_kv_prefill(q, k, v, qw, kw, inv, kc_ref, vc_ref, EPS, ps)

    assert np.array_equal(vc.view(np.uint16), vc_ref.view(np.uint16)), "V cache not bit-exact"
    mask = np.zeros(MS, dtype=bool)
    mask[ps:ps + S] = True
    assert np.all(kc[:, ~mask].view(np.uint16) == sentinel.view(np.uint16)), "K slot outside range written"
    uq = f16_ulp_diff(out, q_ref)
    uk = f16_ulp_diff(kc, kc_ref)
    assert uq.max() <= 1, f"Q max ulp diff {uq.max()}"
    assert uk.max() <= 1, f"K max ulp diff {uk.max()}"
    # Same f32 operation order and correctly rounded sin/cos on both sides:
    # the f16 results are expected bit-identical (an f64 sin/cos rounding tie
    # could flip one in ~1e9).
    assert (uq == 0).mean() > 0.9999 and (uk[:, mask] == 0).mean() > 0.9999


def test_kv_slot_known_answer(gpu):
    """tests/kernels.rs:67-118 (mtp_kv_suffix_write_preserves_prefix_and_unused_tail),
    generalised to D=128 through the fused kernel's V path: HEADS=2, CAPACITY=16,
    START=3, ROWS=5, values i+1; every slot exact, zeros outside [START, START+ROWS)."""
    import torch

    HEADS, CAPACITY, ROWS, START = 2, 16, 5, 3
    values = (np.arange(ROWS * HEADS * D) + 1).astype(np.float16).reshape(ROWS, HEADS, D)
    q = np.zeros((ROWS, HEADS, D), dtype=np.float16)
    ones = np.ones(D, dtype=np.float16)
    inv = oracle.build_inv_freq(THETA)
    kc0 = np.zeros((HEADS, CAPACITY, D), dtype=np.float16)
    vc0 = np.zeros((HEADS, CAPACITY, D), dtype=np.float16)
    _, _, vc = _run_prefill(torch, q, values, values, ones, ones, inv, kc0, vc0, START)
    for head in range(HEADS):
        for pos in range(CAPACITY):
            expected = values[pos - START, head] if START <= pos < START + ROWS else np.zeros(D)
            assert np.array_equal(vc[head, pos].astype(np.float32), expected.astype(np.float32)), (head, pos)


def test_prefill_position_zero_closed_form(gpu):
    """pos 0: RoPE is the identity, so K = f16(x * rsqrt(mean(x^2)+eps) * w) (float64 check)."""
    import torch

    g = rng(11)
    hq, hkv, S = 4, 2, 1
    q, k, v = normal_f16(g, (S, hq, D)), normal_f16(g, (S, hkv, D)), normal_f16(g, (S, hkv, D))
    qw, kw = norm_weight(g), norm_weight(g)
    inv = oracle.build_inv_freq(THETA)
    kc0 = np.zeros((hkv, 4, D), dtype=np.float16)
    out, kc, _ = _run_prefill(torch, q, k, v, qw, kw, inv, kc0, kc0.copy(), 0)
    x = k[0].astype(np.float64)
    ref = x / np.sqrt((x * x).mean(axis=-1, keepdims=True) + EPS) * kw.astype(np.float64)
    assert f16_ulp_diff(kc[:, 0], ref.astype(np.float16)).max() <= 1


@pytest.mark.parametrize("hq,hkv,pos,MS,seed", [
    (32, 8, 4096, 4200, 21),     # config c2 decode step
    (64, 8, 32768, 33792, 22),   # config c4 decode step
    (4, 2, 0, 8, 23),
])
def test_decode_matches_oracle(gpu, hq, hkv, pos, MS, seed):
    import torch

    import grout_amd

    g = rng(seed)
    qkv = normal_f16(g, ((hq + 2 * hkv) * D,))
    qw, kw = norm_weight(g), norm_weight(g)
    inv = oracle.build_inv_freq(THETA)
    kc0 = normal_f16(g, (hkv, MS, D))
    vc0 = normal_f16(g, (hkv, MS, D))
    qout0 = np.full(((hq + hkv), D), np.float16(3.5), dtype=np.float16)

    dqkv, dqw, dkw = _to_dev(torch, qkv), _to_dev(torch, qw), _to_dev(torch, kw)
    dinv = _to_dev(torch, inv)
    dkc, dvc, dqo = _to_dev(torch, kc0), _to_dev(torch, vc0), _to_dev(torch, qout0)
    dpos = torch.tensor([pos], dtype=torch.int32, device="cuda")
    grout_amd.qk_norm_rope_kv_decode(dqkv, dqw, dkw, dinv, dqo, dkc, dvc, dpos, EPS, hq, hkv)
    torch.cuda.synchronize()
    qo, kc, vc = dqo.cpu().numpy(), dkc.cpu().numpy(), dvc.cpu().numpy()

    qo_ref, kc_ref, vc_ref = qout0.copy(), kc0.copy(), vc0.copy()
    oracle.qk_norm_rope_kv_decode(qkv, qw, kw, inv, qo_ref, kc_ref, vc_ref, pos, EPS, hq, hkv)
    assert np.array_equal(vc.view(np.uint16), vc_ref.view(np.uint16))
    assert np.array_equal(qo[hq:].view(np.uint16), qout0[hq:].view(np.uint16)), "rows >= Hq written"
    other = np.ones(MS, dtype=bool)
    other[pos] = False
    assert np.array_equal(kc[:, other].view(np.uint16), kc0[:, other].view(np.uint16))
    assert f16_ulp_diff(qo[:hq], qo_ref[:hq]).max() <= 1
    assert f16_ulp_diff(kc[:, pos], kc_ref[:, pos]).max() <= 1


def test_decode_equals_prefill_row(gpu):
    """A decode step at position p writes what a one-token prefill at p writes."""
    import torch

    import grout_amd

    g = rng(31)
    hq, hkv, MS, pos = 32, 8, 64, 37
    qkv = normal_f16(g, ((hq + 2 * hkv) * D,))
    qw, kw = norm_weight(g), norm_weight(g)
    inv = _to_dev(torch, oracle.build_inv_freq(THETA))
    dqkv = _to_dev(torch, qkv)
    dqw, dkw = _to_dev(torch, qw), _to_dev(torch, kw)
    kc1 = torch.zeros((hkv, MS, D), dtype=torch.float16, device="cuda")
    vc1 = torch.zeros_like(kc1)
    kc2, vc2 = torch.zeros_like(kc1), torch.zeros_like(kc1)
    qo1 = torch.zeros(((hq + hkv), D), dtype=torch.float16, device="cuda")
    dpos = torch.tensor([pos], dtype=torch.int32, device="cuda")
    grout_amd.qk_norm_rope_kv_decode(dqkv, dqw, dkw, inv, qo1, kc1, vc1, dpos, EPS, hq, hkv)
    q = dqkv[: hq * D].view(1, hq, D)
    k = dqkv[hq * D:(hq + hkv) * D].view(1, hkv, D)
    v = dqkv[(hq + hkv) * D:].view(1, hkv, D)
    qo2 = torch.zeros((1, hq, D), dtype=torch.float16, device="cuda")
    grout_amd.qk_norm_rope_kv_prefill(q, k, v, dqw, dkw, inv, qo2, kc2, vc2, EPS, pos)
    torch.cuda.synchronize()
    assert torch.equal(qo1[:hq], qo2[0])
    assert torch.equal(kc1, kc2) and torch.equal(vc1, vc2)
