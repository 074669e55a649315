"""Pins the CPU oracle (oracle/grout_oracle.c) before it is trusted as the checker.

Each oracle function is checked against something that does not restate its
own formula: the reference's KV-slot known-answer test (tests/kernels.rs:67-118),
closed forms, invariants, numpy's f16 conversion, an independent float64
formulation, and torch's CPU scaled_dot_product_attention.  Each check is chosen
so a plausible slip (dropped term, wrong sign or half pairing, wrong index or
stride, transposed operand, wrong split boundary) fails at least one of them.
"""
import math

import numpy as np
import pytest

import oracle
from tests._util import (D, EPS, THETA, f16_ulp_diff, norm_weight, normal_f16, qk_scale_f16_bits,
                         qwen3_tiny_model, rng)

SCALE = 1.0 / math.sqrt(D)


# ------------------------------------------------------------------- f16 --

def test_f16_conversion_matches_numpy():
    g = np.random.default_rng(0)
    x = np.concatenate([
        g.standard_normal(200000).astype(np.float32) * np.float32(3000),
        g.standard_normal(50000).astype(np.float32) * np.float32(1e-5),   # f16 subnormals
        np.float32([0.0, -0.0, 65504, 65519.99, 65520, -65520, 2.0 ** -24, 2.0 ** -25,
                    2.0 ** -25 * 1.0001, 3 * 2.0 ** -26, 6.1035156e-05, np.inf, -np.inf]),
    ])
    with np.errstate(over="ignore"):
        ref = x.astype(np.float16)
    assert np.array_equal(oracle.f32_to_f16(x).view(np.uint16), ref.view(np.uint16))
    allbits = np.arange(65536, dtype=np.uint16).view(np.float16)
    finite = np.isfinite(allbits)
    back = oracle.f16_to_f32(allbits)
    assert np.array_equal(back[finite], allbits[finite].astype(np.float32))
    assert np.all(np.isnan(back[np.isnan(allbits)]))


# -------------------------------------------------------------- inv_freq --

def test_inv_freq_closed_form():
    inv = oracle.build_inv_freq(THETA)
    assert inv.shape == (64,) and inv[0] == 1.0
    j = np.arange(64)
    exact = THETA ** (-(2.0 * j) / D)
    assert np.allclose(inv, exact, rtol=3e-7, atol=0)
    assert abs(inv[32] - 1e-3) < 1e-9  # theta^(-1/2)
    assert np.all(np.diff(inv) < 0)
    # Qwen3 default theta 1e4 gives the textbook 10000^(-2j/d) table.
    inv4 = oracle.build_inv_freq(1e4)
    assert np.allclose(inv4, 1e4 ** (-(2.0 * j) / D), rtol=3e-7)


# ------------------------------------------------------- fused norm/RoPE --

def _rope_f64(x, w, inv, pos):
    """Independent float64 formulation: RMSNorm then rotate each (j, j+64) pair
    as a complex number by the f32 angle f32(pos)*inv_freq[j]."""
    x = x.astype(np.float64)
    n = x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + EPS) * w.astype(np.float64)
    theta = (np.float32(pos) * inv).astype(np.float64)
    z = (n[..., :64] + 1j * n[..., 64:]) * np.exp(1j * theta)
    return np.concatenate([z.real, z.imag], axis=-1)


def _prefill(q, k, v, qw, kw, ps, MS, fill=0.0):
    hkv = k.shape[1]
    kc = np.full((hkv, MS, D), fill, dtype=np.float16)
    vc = np.full((hkv, MS, D), fill, dtype=np.float16)
    inv = oracle.build_inv_freq(THETA)
    qo = oracle.qk_norm_rope_kv_prefill(q, k, v, qw, kw, inv, kc, vc, EPS, ps)
    return qo, kc, vc


def test_kv_slot_known_answer():
    """Reference KAT tests/kernels.rs:67-118 (HEADS=2, CAPACITY=16, START=3, ROWS=5,
    values i+1) on the fused op's V path, D=128: every slot exact, zeros elsewhere."""
    HEADS, CAPACITY, ROWS, START = 2, 16, 5, 3
    values = (np.arange(ROWS * HEADS * D) + 1).astype(np.float16).reshape(ROWS, HEADS, D)
    ones = np.ones(D, dtype=np.float16)
    _, _, vc = _prefill(np.zeros_like(values), values, values, ones, ones, START, CAPACITY)
    for head in range(HEADS):
        for pos in range(CAPACITY):
            exp = values[pos - START, head] if START <= pos < START + ROWS else np.zeros(D)
            assert np.array_equal(vc[head, pos].astype(np.float32), exp.astype(np.float32))


@pytest.mark.parametrize("ps,seed", [(0, 1), (5, 2), (32700, 3)])
def test_norm_rope_matches_float64(ps, seed):
    g = rng(seed)
    S, hq, hkv = 9, 4, 2
    q, k, v = normal_f16(g, (S, hq, D)), normal_f16(g, (S, hkv, D)), normal_f16(g, (S, hkv, D))
    qw, kw = norm_weight(g), norm_weight(g)
    qo, kc, vc = _prefill(q, k, v, qw, kw, ps, ps + S + 3)
    inv = oracle.build_inv_freq(THETA)
    pos = ps + np.arange(S)
    qr = np.stack([_rope_f64(q[s], qw, inv, pos[s]) for s in range(S)])
    kr = np.stack([_rope_f64(k[s], kw, inv, pos[s]) for s in range(S)])
    assert f16_ulp_diff(qo, qr.astype(np.float16)).max() <= 1
    assert f16_ulp_diff(kc[:, ps:ps + S].transpose(1, 0, 2), kr.astype(np.float16)).max() <= 1
    assert np.array_equal(vc[:, ps:ps + S].transpose(1, 0, 2), v)


def test_rope_single_element_pairs_j_with_j_plus_64():
    """x = a*e_0: n_0 = sqrt(128)*w_0, y_0 = n_0 cos(pos), y_64 = n_0 sin(pos)
    (inv_freq[0] = 1); every other element stays 0.  Pins the half pairing and
    the rotation direction."""
    x = np.zeros((1, 1, D), dtype=np.float16)
    x[0, 0, 0] = 3.0
    ones = np.ones(D, dtype=np.float16)
    pos = 2
    qo, _, _ = _prefill(x, x[:, :1], x[:, :1], ones, ones, pos, pos + 1)
    n0 = 3.0 / math.sqrt(9.0 / 128 + EPS)
    assert qo[0, 0, 0] == np.float16(n0 * math.cos(2.0))
    assert qo[0, 0, 64] == np.float16(n0 * math.sin(2.0))
    assert np.count_nonzero(qo) == 2


def test_rope_relative_position_invariance():
    """<rope(q,a), rope(k,b)> depends only on a-b (same rotation for q and k)."""
    g = rng(4)
    q = normal_f16(g, (1, 1, D))
    k = normal_f16(g, (1, 1, D))
    ones = np.ones(D, dtype=np.float16)

    def dot(a, b):
        qa, _, _ = _prefill(q, k, k, ones, ones, a, a + 1)
        _, kb, _ = _prefill(q, k, k, ones, ones, b, b + 1)
        return float(np.dot(qa[0, 0].astype(np.float64), kb[0, b].astype(np.float64)))

    d1, d2, d3 = dot(10, 3), dot(110, 103), dot(3, 10)
    assert abs(d1 - d2) < 0.05 and abs(d1 - d3) > 0.05


def test_decode_equals_prefill_row():
    g = rng(5)
    hq, hkv, MS, pos = 8, 2, 40, 33
    qkv = normal_f16(g, ((hq + 2 * hkv) * D,))
    qw, kw = norm_weight(g), norm_weight(g)
    inv = oracle.build_inv_freq(THETA)
    qo = np.zeros((hq + hkv, D), dtype=np.float16)
    kc, vc = np.zeros((hkv, MS, D), np.float16), np.zeros((hkv, MS, D), np.float16)
    oracle.qk_norm_rope_kv_decode(qkv, qw, kw, inv, qo, kc, vc, pos, EPS, hq, hkv)
    q = qkv[:hq * D].reshape(1, hq, D)
    k = qkv[hq * D:(hq + hkv) * D].reshape(1, hkv, D)
    v = qkv[(hq + hkv) * D:].reshape(1, hkv, D)
    qo2, kc2, vc2 = _prefill(q, k, v, qw, kw, pos, MS)
    assert np.array_equal(qo[:hq], qo2[0]) and np.all(qo[hq:] == 0)
    assert np.array_equal(kc, kc2) and np.array_equal(vc, vc2)


# ------------------------------------------------------ prefill attention --

def _attn_f64(q, kc, vc, scale, kv_len, qs):
    S, hq, _ = q.shape
    hkv = kc.shape[0]
    G = hq // hkv
    out = np.zeros((S, hq, D))
    for h in range(hq):
        K = kc[h // G, :kv_len].astype(np.float64)
        V = vc[h // G, :kv_len].astype(np.float64)
        s = q[:, h].astype(np.float64) @ K.T * scale
        pos = qs + np.arange(S)[:, None]
        s = np.where(np.arange(kv_len)[None, :] <= pos, s, -np.inf)
        p = np.exp(s - s.max(axis=1, keepdims=True))
        out[:, h] = (p / p.sum(axis=1, keepdims=True)) @ V
    return out


@pytest.mark.parametrize("hq,hkv,S,qs,MS", [(4, 2, 17, 0, 17), (4, 2, 9, 5, 20),
                                            (6, 3, 33, 0, 40), (2, 2, 64, 0, 64)])
def test_attention_matches_float64_bruteforce(hq, hkv, S, qs, MS):
    g = rng(6)
    q, kc, vc = normal_f16(g, (S, hq, D)), normal_f16(g, (hkv, MS, D)), normal_f16(g, (hkv, MS, D))
    out = oracle.attn_prefill_f32(q, kc, vc, SCALE, qs + S, qs)
    ref = _attn_f64(q, kc, vc, SCALE, qs + S, qs)
    assert np.max(np.abs(out - ref)) < 2e-5


def test_attention_matches_torch_sdpa():
    torch = pytest.importorskip("torch")
    g = rng(7)
    S, hq, hkv = 48, 8, 2
    q, kc, vc = normal_f16(g, (S, hq, D)), normal_f16(g, (hkv, S, D)), normal_f16(g, (hkv, S, D))
    out = oracle.attn_prefill_f32(q, kc, vc, SCALE, S, 0)
    tq = torch.from_numpy(q.astype(np.float32)).permute(1, 0, 2)
    tk = torch.from_numpy(kc.astype(np.float32)).repeat_interleave(hq // hkv, dim=0)
    tv = torch.from_numpy(vc.astype(np.float32)).repeat_interleave(hq // hkv, dim=0)
    ref = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, is_causal=True,
                                                           scale=SCALE)
    assert np.max(np.abs(out - ref.permute(1, 0, 2).numpy())) < 2e-5


def test_attention_special_cases():
    g = rng(8)
    S, hq, hkv = 12, 4, 2
    q, kc, vc = normal_f16(g, (S, hq, D)), normal_f16(g, (hkv, S, D)), normal_f16(g, (hkv, S, D))
    out = oracle.attn_prefill_f32(q, kc, vc, SCALE, S, 0)
    # Row 0 sees only key 0.
    for h in range(hq):
        assert np.array_equal(out[0, h], vc[h // 2, 0].astype(np.float32))
    # Identical keys: uniform weights -> causal prefix mean of V.
    kc_same = np.repeat(kc[:, :1], S, axis=1)
    o2 = oracle.attn_prefill_f32(q, kc_same, vc, SCALE, S, 0)
    for m in range(S):
        assert np.allclose(o2[m, 0], vc[0, :m + 1].astype(np.float64).mean(0), atol=1e-5)
    # One dominant key: the row returns that V row.
    kc_dom = np.zeros_like(kc)
    qd = np.zeros_like(q)
    qd[:, :, 0] = 8.0
    kc_dom[:, 3, 0] = 64.0
    o3 = oracle.attn_prefill_f32(qd, kc_dom, vc, SCALE, S, 0)
    assert np.allclose(o3[5:, 0], vc[0, 3].astype(np.float32), atol=1e-6)


def test_attention_chunked_equals_full_and_row_sampling():
    g = rng(9)
    S, hq, hkv = 40, 4, 2
    q, kc, vc = normal_f16(g, (S, hq, D)), normal_f16(g, (hkv, S, D)), normal_f16(g, (hkv, S, D))
    full = oracle.attn_prefill_f32(q, kc, vc, SCALE, S, 0)
    part = oracle.attn_prefill_f32(np.ascontiguousarray(q[25:]), kc, vc, SCALE, S, 25)
    assert np.array_equal(full[25:], part)
    samp = oracle.attn_prefill_f32(q, kc, vc, SCALE, S, 0, row_begin=3, row_step=7)
    rows = np.arange(3, S, 7)
    assert np.array_equal(samp[rows], full[rows])
    others = np.setdiff1d(np.arange(S), rows)
    assert np.all(samp[others] == 0)


# ---------------------------------------------------------- split decode --

def test_split_ranges_partition_tiles():
    for s_kv in (1, 31, 32, 33, 4097, 32769):
        for ns in (1, 3, 16, 64, 200):
            tiles = -(-s_kv // 32)
            covered = []
            for s in range(ns):
                b, e = oracle.decode_split_range(s_kv, 32, ns, s)
                covered.extend(range(b, max(b, e)))
            assert covered == list(range(tiles)), (s_kv, ns)


def _dec_case(seed, hkv, G, MS):
    g = rng(seed)
    return (normal_f16(g, (hkv, G, D)), normal_f16(g, (hkv, MS, D)), normal_f16(g, (hkv, MS, D)))


@pytest.mark.parametrize("ns", [1, 5, 16])
def test_split_merge_matches_float64_decode(ns):
    qg, kc, vc = _dec_case(10, 2, 4, 300)
    pos = 260
    att, lse = oracle.attn_decode_split(qg, kc, vc, qk_scale_f16_bits(), pos, 32, ns)
    out = oracle.attn_decode_merge(att, lse, 4).astype(np.float32)
    scale = float(np.array([qk_scale_f16_bits()], np.uint16).view(np.float16)[0])
    q = qg.reshape(1, 8, D)
    ref = _attn_f64(q, kc, vc, scale, pos + 1, pos).reshape(2, 4, D)
    assert np.max(np.abs(out - ref)) < 2e-3
    # Each non-empty partial is itself the softmax over its token range.
    s_kv = pos + 1
    for s in range(ns):
        b, e = oracle.decode_split_range(s_kv, 32, ns, s)
        if b >= e:
            continue
        lo, hi = b * 32, min(e * 32, s_kv)
        for h in range(2):
            K = kc[h, lo:hi].astype(np.float64)
            logits = qg[h].astype(np.float64) @ K.T * scale
            p = np.exp(logits - logits.max(1, keepdims=True))
            part = p / p.sum(1, keepdims=True) @ vc[h, lo:hi].astype(np.float64)
            rows = slice(s * 4, s * 4 + 4)
            assert np.max(np.abs(att[h, rows].astype(np.float64) - part)) < 2e-3
            lse_ref = (np.log(np.exp(logits).sum(1))) / math.log(2)
            assert np.max(np.abs(lse[h, rows] - lse_ref)) < 1e-4


def test_fused_split_ranges_partition_tokens():
    """The fused decode step's boundaries (not the reference's): contiguous
    16-token-aligned ranges covering [0, s_kv), sizes within one sub-chunk."""
    for s_kv in (1, 15, 16, 17, 4097, 32769):
        for ns in (1, 3, 16, 32, 200):
            ranges = [oracle.decode_split_range_fused(s_kv, ns, s) for s in range(ns)]
            covered = []
            for b, e in ranges:
                assert b % 16 == 0 and b <= e
                covered.extend(range(b, e))
            assert covered == list(range(s_kv)), (s_kv, ns)
            subs = [-(-(e - b) // 16) for b, e in ranges]
            assert max(subs) - min(subs) <= 1, (s_kv, ns)
            assert ranges[-1][1] == s_kv  # the last split holds the newest token


@pytest.mark.parametrize("ns", [1, 5, 16])
def test_fused_ranges_split_merge_matches_float64_decode(ns):
    """The same split arithmetic on the fused boundaries: partials are the
    softmax over their token ranges and the merge is the full attention."""
    qg, kc, vc = _dec_case(13, 2, 4, 300)
    pos = 260
    att, lse = oracle.attn_decode_split(qg, kc, vc, qk_scale_f16_bits(), pos, 32, ns,
                                        fused_ranges=True)
    out = oracle.attn_decode_merge(att, lse, 4).astype(np.float32)
    scale = float(np.array([qk_scale_f16_bits()], np.uint16).view(np.float16)[0])
    ref = _attn_f64(qg.reshape(1, 8, D), kc, vc, scale, pos + 1, pos).reshape(2, 4, D)
    assert np.max(np.abs(out - ref)) < 2e-3
    for s in range(ns):
        lo, hi = oracle.decode_split_range_fused(pos + 1, ns, s)
        if lo >= hi:
            assert np.all(lse[:, s * 4:s * 4 + 4] == np.float32(-1e30))
            continue
        for h in range(2):
            logits = qg[h].astype(np.float64) @ kc[h, lo:hi].astype(np.float64).T * scale
            p = np.exp(logits - logits.max(1, keepdims=True))
            part = p / p.sum(1, keepdims=True) @ vc[h, lo:hi].astype(np.float64)
            rows = slice(s * 4, s * 4 + 4)
            assert np.max(np.abs(att[h, rows].astype(np.float64) - part)) < 2e-3
            lse_ref = (np.log(np.exp(logits).sum(1))) / math.log(2)
            assert np.max(np.abs(lse[h, rows] - lse_ref)) < 1e-4


def test_empty_split_and_single_key():
    qg, kc, vc = _dec_case(11, 2, 4, 64)
    att, lse = oracle.attn_decode_split(qg, kc, vc, qk_scale_f16_bits(), 0, 32, 4)
    assert np.all(att[:, 4:] == 0) and np.all(lse[:, 4:] == np.float32(-1e30))
    out = oracle.attn_decode_merge(att, lse, 4)
    for h in range(2):
        assert np.array_equal(out[h], np.repeat(vc[h, :1], 4, axis=0))


def test_merge_closed_forms():
    hkv, G, ns = 1, 2, 2
    att = np.zeros((hkv, ns * G, D), dtype=np.float16)
    att[0, 0:2] = 1.0   # split 0
    att[0, 2:4] = 4.0   # split 1
    lse = np.zeros((hkv, ns * G), dtype=np.float32)
    out = oracle.attn_decode_merge(att, lse, G)
    assert np.all(out == np.float16(2.5))  # equal LSE -> mean
    lse[0, 2:4] = 1.0  # split 1 twice as heavy (log2 units)
    out = oracle.attn_decode_merge(att, lse, G)
    assert np.allclose(out.astype(np.float32), (1.0 + 2 * 4.0) / 3, atol=2e-3)


def test_split_invariance_oracle():
    qg, kc, vc = _dec_case(12, 2, 8, 1000)
    outs = []
    for ns in (1, 4, 31):
        att, lse = oracle.attn_decode_split(qg, kc, vc, qk_scale_f16_bits(), 999, 32, ns)
        outs.append(oracle.attn_decode_merge(att, lse, 8).astype(np.float32))
    assert np.max(np.abs(outs[1] - outs[0])) < 2e-3
    assert np.max(np.abs(outs[2] - outs[0])) < 2e-3


def test_decode_scale_is_f16_rounded():
    """src/model.rs:3427: the decode scale is f16(1/sqrt(128)) = 0.08837890625."""
    assert qk_scale_f16_bits() == 0x2DA8 == oracle.f16_bits(SCALE)
    assert float(np.array([0x2DA8], np.uint16).view(np.float16)[0]) == 0.08837890625


def test_kv_cache_update_seq_reference_kat():
    """tests/kernels.rs:67-118 (mtp_kv_suffix_write_preserves_prefix_and_unused_tail):
    HEADS=2, CAPACITY=16, D=4, ROWS=5, START=3, incoming values i+1; slot
    [h, pos, d] = values[((pos-START)*HEADS + h)*D + d] inside the range, the
    zero-initialised prefix and tail stay 0."""
    HEADS, CAP, D, ROWS, START = 2, 16, 4, 5, 3
    values = (np.arange(ROWS * HEADS * D) + 1).astype(np.float16).reshape(ROWS, HEADS, D)
    k = np.zeros((HEADS, CAP, D), np.float16)
    v = np.zeros((HEADS, CAP, D), np.float16)
    oracle.kv_cache_update_seq(values, values, k, v, START)
    flat = values.reshape(-1)
    for h in range(HEADS):
        for pos in range(CAP):
            for d in range(D):
                exp = flat[((pos - START) * HEADS + h) * D + d] if START <= pos < START + ROWS else 0
                assert k[h, pos, d] == exp and v[h, pos, d] == exp


def test_kv_cache_update_seq_leaves_other_slots():
    """Rows outside [start, start+S) keep whatever the cache held (sentinels)."""
    g = np.random.default_rng(5)
    Hkv, MS, D, S, start = 3, 40, 128, 7, 29
    nk = g.standard_normal((S, Hkv, D)).astype(np.float16)
    nv = g.standard_normal((S, Hkv, D)).astype(np.float16)
    k = np.full((Hkv, MS, D), 7.0, np.float16)
    v = np.full((Hkv, MS, D), -3.0, np.float16)
    oracle.kv_cache_update_seq(nk, nv, k, v, start)
    assert np.array_equal(k[:, start:start + S], nk.transpose(1, 0, 2))
    assert np.array_equal(v[:, start:start + S], nv.transpose(1, 0, 2))
    assert (k[:, :start] == 7).all() and (k[:, start + S:] == 7).all()
    assert (v[:, :start] == -3).all() and (v[:, start + S:] == -3).all()


# ------------------------------------------------------- split-K prefill --

def _split_range_tiles(b, bm, bn, ns, s, kv_len, qs):
    """Split s of q block b: KV tiles [s*tps, min(s*tps+tps, tc)) with
    tc = ceil(min(qs+(b+1)*bm, kv_len)/bn), tps = ceil(tc/ns)
    (src/kernels.rs:2036-2043), computed here from the formula's text."""
    tc = -(-min(qs + (b + 1) * bm, kv_len) // bn)
    tps = -(-tc // ns)
    return s * tps, min(s * tps + tps, tc)


def _prefill_split_f64(q, kc, vc, scale, kv_len, qs, bm, bn, gr, ns):
    """Independent float64 statement of every partial: the softmax of each
    (row, head) over the causal keys of its split's range, its LSE in log2
    units, and the reference layout [tile, s*BM*GR + bm*GR + g]."""
    S, hq, _ = q.shape
    hkv = kc.shape[0]
    nb = -(-S // bm)
    ngrp = hq // gr
    att = np.zeros((nb * ngrp, ns * bm * gr, D))
    lse = np.full((nb * ngrp, ns * bm * gr), np.nan)
    for b in range(nb):
        for s in range(ns):
            t0, t1 = _split_range_tiles(b, bm, bn, ns, s, kv_len, qs)
            lo, hi = t0 * bn, min(t1 * bn, kv_len)
            for i in range(bm):
                row = b * bm + i
                pos = qs + row
                for h in range(hq):
                    tile, r = b * ngrp + h // gr, s * bm * gr + i * gr + h % gr
                    kv = h // (hq // hkv)
                    keys = np.arange(lo, min(hi, pos + 1))
                    if len(keys) == 0:
                        lse[tile, r] = -np.inf  # empty or fully masked: zero weight
                        continue
                    qv = q[row, h].astype(np.float64) if row < S else np.zeros(D)
                    z = kc[kv, keys].astype(np.float64) @ qv * scale
                    w = np.exp(z - z.max())
                    att[tile, r] = w / w.sum() @ vc[kv, keys].astype(np.float64)
                    lse[tile, r] = (z.max() + np.log(w.sum())) / math.log(2)
    return att, lse


@pytest.mark.parametrize("S,qs,kv_len,hq,hkv,bm,bn,gr,ns", [
    (40, 0, 40, 4, 2, 32, 32, 2, 3),     # ragged q_len, GROUP = q group size
    (64, 0, 64, 4, 2, 32, 16, 1, 4),     # GROUP 1, BN not the kernel tile
    (33, 7, 40, 6, 3, 64, 32, 2, 2),     # query_start > 0, padded rows
    (48, 0, 48, 8, 2, 16, 8, 4, 5),      # small tiles, many splits
])
def test_prefill_split_partials_match_float64(S, qs, kv_len, hq, hkv, bm, bn, gr, ns):
    g = rng(30)
    MS = kv_len + 3
    q, kc, vc = normal_f16(g, (S, hq, D)), normal_f16(g, (hkv, MS, D)), normal_f16(g, (hkv, MS, D))
    att, lse = oracle.attn_prefill_split(q, kc, vc, SCALE, kv_len, qs, bm, bn, gr, ns)
    att64, lse64 = _prefill_split_f64(q, kc, vc, SCALE, kv_len, qs, bm, bn, gr, ns)
    live = np.isfinite(lse64)
    assert live.any()
    assert np.max(np.abs(att.astype(np.float64)[live] - att64[live])) < 2e-3
    assert np.max(np.abs(lse[live] - lse64[live])) < 1e-4
    # Empty ranges store O = 0, LSE = -1e30 exactly; ranges whose keys are all
    # masked for a row (the split starts past its position) carry a finite
    # partial but an LSE below -1e28, i.e. weight 0 in the merge.
    assert np.all(lse[~live] < -1e28)
    out = oracle.attn_prefill_split_merge(att, lse, hq, S, bm, gr, ns).astype(np.float32)
    ref = _attn_f64(q, kc, vc, SCALE, kv_len, qs)
    assert np.max(np.abs(out - ref)) < 2e-3


def test_prefill_split_empty_splits_and_invariance():
    g = rng(31)
    S, hq, hkv = 20, 4, 2
    q, kc, vc = normal_f16(g, (S, hq, D)), normal_f16(g, (hkv, S, D)), normal_f16(g, (hkv, S, D))
    # One 32-row block over 20 keys: tc = 1 tile of 32, so splits 1.. are empty.
    att, lse = oracle.attn_prefill_split(q, kc, vc, SCALE, S, 0, 32, 32, 2, 4)
    ns_m = 32 * 2
    assert np.all(att[:, ns_m:] == 0) and np.all(lse[:, ns_m:] == np.float32(-1e30))
    outs = []
    for ns in (1, 2, 7):
        a, l = oracle.attn_prefill_split(q, kc, vc, SCALE, S, 0, 32, 4, 2, ns)
        outs.append(oracle.attn_prefill_split_merge(a, l, hq, S, 32, 2, ns).astype(np.float32))
    full = oracle.attn_prefill_f32(q, kc, vc, SCALE, S, 0)
    for o in outs:
        assert np.max(np.abs(o - full)) < 2e-3
    # Row 0 of every head sees key 0 only: exactly V[0] through the merge.
    for h in range(hq):
        assert np.array_equal(outs[2][0, h], vc[h // 2, 0].astype(np.float32))


def test_prefill_split_merge_closed_forms():
    bm, gr, ns, hq, S = 16, 1, 2, 1, 16
    att = np.zeros((1, ns * bm * gr, D), dtype=np.float16)
    att[0, :bm] = 1.0      # split 0
    att[0, bm:] = 4.0      # split 1
    lse = np.zeros((1, ns * bm * gr), dtype=np.float32)
    out = oracle.attn_prefill_split_merge(att, lse, hq, S, bm, gr, ns)
    assert np.all(out == np.float16(2.5))  # equal LSE -> mean
    lse[0, bm:] = 1.0  # split 1 twice as heavy (log2 units)
    out = oracle.attn_prefill_split_merge(att, lse, hq, S, bm, gr, ns)
    assert np.allclose(out.astype(np.float32), (1.0 + 2 * 4.0) / 3, atol=2e-3)
    # Layout: row r = bm*GROUP + g of tile b*ngroups + hg is (row b*BM+bm, head hg*GROUP+g).
    bm, gr, hq, S = 2, 2, 4, 3
    att = np.zeros((2 * 2, bm * gr, D), dtype=np.float16)
    for tile in range(4):
        for r in range(bm * gr):
            att[tile, r] = tile * 10 + r
    lse = np.zeros((4, bm * gr), dtype=np.float32)
    out = oracle.attn_prefill_split_merge(att, lse, hq, S, bm, gr, 1)
    for row in range(S):
        for h in range(hq):
            b, i, hg, gg = row // bm, row % bm, h // gr, h % gr
            assert out[row, h, 0] == (b * 2 + hg) * 10 + i * gr + gg


# ------------------------------------------------------ decode-layer ops --
# add_rms_norm_decode_raw_f16 (src/kernels.rs:3076-3216), the cuBLAS GemvInPlace
# of the decode graph (src/cublas.rs:572-607) and the two-stage greedy argmax
# (src/kernels.rs:345-505).

def _f16_ulp(v):
    """Spacing of the f16 grid at |v| (normal range; 2^-24 below it)."""
    a = np.abs(np.asarray(v, dtype=np.float64))
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -14)))
    return 2.0 ** (e - 10)


@pytest.mark.parametrize("n,eps,seed", [(5120, 1e-6, 1), (4096, 1e-6, 2), (40, 0.5, 3),
                                        (8, 1e-6, 4), (32768, 1e-6, 5)])
def test_add_rms_norm_against_float64(n, eps, seed):
    g = rng(900 + seed)
    r, x = normal_f16(g, n, 2.0), normal_f16(g, n, 0.5)
    w = (1.0 + 0.1 * g.standard_normal(n)).astype(np.float16)
    out, res = oracle.add_rms_norm(r, x, w, eps)
    c = r.astype(np.float64) + x.astype(np.float64)
    assert np.all(f16_ulp_diff(res, c.astype(np.float16)) <= 1)
    assert np.mean(res == c.astype(np.float16)) > 0.999
    inv = 1.0 / np.sqrt(np.mean(c * c) + eps)
    exp = c * inv * w.astype(np.float64)
    # The f32 sum of n positive squares is within n * 2^-24 relative, so inv is
    # within (n/2 + 2) * 2^-24; two more f32 roundings and the f16 rounding.
    rel = (n / 2 + 6) * 2.0 ** -24
    assert np.all(np.abs(out.astype(np.float64) - exp) <= _f16_ulp(exp) * 0.5 + rel * np.abs(exp))
    assert np.mean(out == exp.astype(np.float16)) > 0.99


def test_add_rms_norm_closed_forms():
    n = 1024
    h = np.float16
    # residual + x = 1 everywhere, w = 1, eps = 3: inv = 1/sqrt(1 + 3) = 0.5.  A
    # mean over n-1, eps outside the sqrt or a dropped residual all move it.
    out, res = oracle.add_rms_norm(np.full(n, 0.75, h), np.full(n, 0.25, h), np.ones(n, h), 3.0)
    assert np.all(res == h(1.0)) and np.all(out == h(0.5))
    # The weight multiplies elementwise, the residual output is the raw sum.
    w = np.arange(n, dtype=np.float64).astype(h) / h(64)
    out, res = oracle.add_rms_norm(np.full(n, -3.0, h), np.full(n, 1.0, h), w, 0.0)
    assert np.all(res == h(-2.0)) and np.array_equal(out, (-w.astype(np.float64)).astype(h))
    # eps = 0: the output is invariant under power-of-two scaling of the inputs.
    g = rng(910)
    r, x, wn = normal_f16(g, n), normal_f16(g, n), normal_f16(g, n)
    o1, r1 = oracle.add_rms_norm(r, x, wn, 0.0)
    o2, r2 = oracle.add_rms_norm(r * h(8), x * h(8), wn, 0.0)
    assert np.array_equal(o1, o2) and np.array_equal(r2, r1 * h(8))


@pytest.mark.parametrize("m,k,seed", [(300, 512, 1), (64, 5120, 2), (17, 8, 3), (5, 8192, 4)])
def test_gemv_against_float64(m, k, seed):
    g = rng(920 + seed)
    w = normal_f16(g, (m, k), 1.0 / math.sqrt(k))
    x = normal_f16(g, k)
    out = oracle.gemv_f16(w, x)
    w64, x64 = w.astype(np.float64), x.astype(np.float64)
    exp = w64 @ x64
    # f32 accumulation of exact f16 products: |err| <= k * 2^-24 * sum|w x|,
    # plus half an f16 ulp for the final rounding.
    bound = _f16_ulp(exp) * 0.5 + k * 2.0 ** -24 * (np.abs(w64) @ np.abs(x64))
    assert np.all(np.abs(out.astype(np.float64) - exp) <= bound)


def test_gemv_closed_forms():
    # A row-selection matrix (m != k): out[i] = x[perm[i]] exactly; reading the
    # weight transposed or with the wrong row stride picks other entries.
    m, k = 40, 24
    g = rng(930)
    perm = g.integers(0, k, m)
    w = np.zeros((m, k), np.float16)
    w[np.arange(m), perm] = 1.0
    x = normal_f16(g, k)
    assert np.array_equal(oracle.gemv_f16(w, x), x[perm])
    # Linearity: scaling x by a power of two scales the output exactly.
    w = normal_f16(g, (m, 256), 0.0625)
    x = normal_f16(g, 256)
    assert np.array_equal(oracle.gemv_f16(w, x * np.float16(4)),
                          (oracle.gemv_f16(w, x).astype(np.float32) * 4).astype(np.float16))
    # All-ones weight: the sum of x (exact in f32 for these small integers).
    xi = g.integers(-8, 9, 512).astype(np.float16)
    assert oracle.gemv_f16(np.ones((3, 512), np.float16), xi)[0] == np.float16(xi.astype(np.float64).sum())


def test_argmax_against_numpy():
    g = rng(940)
    for n in (1, 7, 2048, 2049, 151936):
        lg = normal_f16(g, n, 4.0)
        assert oracle.argmax_f16(lg) == int(np.argmax(lg))
    n = 151936
    lg = normal_f16(g, n)
    lg[[5000, 90000, 150000]] = np.float16(30.0)   # ties across blocks: lowest index
    assert oracle.argmax_f16(lg) == 5000
    lg[4000] = np.float16(np.nan)                  # NaN is never chosen
    lg[100] = np.float16(-np.inf)
    assert oracle.argmax_f16(lg) == 5000 == int(np.nanargmax(lg))
    assert oracle.argmax_f16(np.full(3000, -np.inf, np.float16)) == 0
    assert oracle.argmax_f16(np.full(3000, np.nan, np.float16)) == 0
    nanfirst = np.array([np.nan, 1.0, 3.0, 3.0, 2.0], np.float16)
    assert oracle.argmax_f16(nanfirst) == 2


def test_silu_mul_against_float64():
    g = rng(950)
    gate = np.concatenate([normal_f16(g, 20000, 4.0),
                           np.float16([0.0, -0.0, 30.0, -30.0, 11.0, -17.0, 65504, -65504])])
    up = normal_f16(g, gate.shape[0])
    out = oracle.silu_mul(gate, up)
    g64, u64 = gate.astype(np.float64), up.astype(np.float64)
    with np.errstate(over="ignore"):
        exp = g64 / (1.0 + np.exp(-g64)) * u64
    finite = np.isfinite(exp) & (np.abs(exp) < 65504)
    assert np.all(f16_ulp_diff(out[finite], exp[finite].astype(np.float16)) <= 1)
    assert np.mean(out[finite] == exp[finite].astype(np.float16)) > 0.999
    # silu(0) = 0, silu(g) -> g for large g, -> 0 for very negative g.
    one = np.ones(4, np.float16)
    assert np.array_equal(oracle.silu_mul(np.float16([0.0, 30.0, -30.0, -100.0]), one),
                          np.float16([0.0, 30.0, -0.0, -0.0]))


def _qwen3_step_f64(m, token, pos):
    """Independent float64 Qwen3 decode step (no f16 intermediates): RMSNorm,
    merged QKV, per-head QK norm + RoPE, causal attention over [0, pos],
    residual adds, SwiGLU MLP, final norm, lm_head.  Returns logits and the
    updated caches."""
    f = lambda a: a.astype(np.float64)  # noqa: E731
    hq, hkv = m["num_q_heads"], m["num_kv_heads"]
    G = hq // hkv
    inv = oracle.build_inv_freq(THETA)
    scale = float(np.array([qk_scale_f16_bits()], np.uint16).view(np.float16)[0])

    def rms(x, w):
        return x / np.sqrt(np.mean(x * x) + EPS) * f(w)

    h = f(m["embed_tokens"][token])
    caches = []
    for L in m["layers"]:
        qkv = f(L["qkv_proj"]) @ rms(h, L["input_norm"])
        q = _rope_f64(qkv[:hq * D].reshape(hq, D), L["q_norm"], inv, pos)
        k = _rope_f64(qkv[hq * D:(hq + hkv) * D].reshape(hkv, D), L["k_norm"], inv, pos)
        v = qkv[(hq + hkv) * D:].reshape(hkv, D)
        kc, vc = f(L["k_cache"]), f(L["v_cache"])
        kc[:, pos], vc[:, pos] = k, v
        caches.append((kc, vc))
        o = np.zeros((hq, D))
        for hd in range(hq):
            s = kc[hd // G, :pos + 1] @ q[hd] * scale
            p = np.exp(s - s.max())
            o[hd] = (p / p.sum()) @ vc[hd // G, :pos + 1]
        h = h + f(L["o_proj"]) @ o.reshape(-1)
        gu = f(L["gate_up_proj"]) @ rms(h, L["post_attn_norm"])
        gt, up = np.split(gu, 2)
        h = h + f(L["down_proj"]) @ (gt / (1.0 + np.exp(-gt)) * up)
    return f(m["lm_head"]) @ rms(h, m["final_norm"]), caches


def test_qwen3_decode_step_against_float64():
    """The oracle's token step (its ops composed in the graph's order,
    src/model.rs:3118-3648) against the float64 formulation: logits within
    1% of their spread, caches written at `pos` within 1 f16 ulp of the
    float64 K/V (layer 0) and within the f16 noise of later layers.  A
    dropped residual add, swapped norms, gate/up swapped or a transposed
    projection moves the logits by O(their spread)."""
    m = qwen3_tiny_model(960)
    pos, token = 20, 123
    ref_logits, ref_caches = _qwen3_step_f64(m, token, pos)
    logits, nxt = oracle.qwen3_decode_step(m, token, pos, block_n=32, num_splits=3)
    spread = ref_logits.std()
    err = np.abs(logits.astype(np.float64) - ref_logits)
    assert spread > 1.0 and err.max() < 0.01 * spread, (err.max(), spread)
    assert nxt == int(np.argmax(logits))
    for li in range(len(m["layers"])):
        for c in range(2):
            got = m["layers"][li][("k_cache", "v_cache")[c]]
            d = np.abs(got[:, pos].astype(np.float64) - ref_caches[li][c][:, pos])
            # f16 rounding of qkv before the norm: a few 1e-3 on O(1) rows.
            assert d.max() < (5e-3 if li == 0 else 2e-2), (li, c, d.max())
            assert np.array_equal(got[:, :pos], ref_caches[li][c][:, :pos].astype(np.float16))
