"""The committed golden fixtures (tests/golden/*.npz, written by
tests/golden/make_golden.py from the oracle) are reproduced bit-exactly by the
oracle: a change to the oracle's arithmetic shows up here."""
import math
import os

import numpy as np

import oracle

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
D = 128


def load(name):
    return np.load(os.path.join(GOLD, name))  # allow_pickle=False (default)


def f16(a):
    return np.ascontiguousarray(a).view(np.float16)


def test_norm_rope_prefill_fixture():
    z = load("qk_norm_rope_prefill.npz")
    q, k, v = f16(z["q"]), f16(z["k"]), f16(z["v"])
    hkv, MS = k.shape[1], f16(z["k_cache"]).shape[1]
    kc = np.zeros((hkv, MS, D), np.float16)
    vc = np.zeros((hkv, MS, D), np.float16)
    qo = oracle.qk_norm_rope_kv_prefill(q, k, v, f16(z["q_weight"]), f16(z["k_weight"]),
                                        z["inv_freq"], kc, vc, float(z["eps"]),
                                        int(z["position_start"]))
    assert np.array_equal(qo.view(np.uint16), z["q_out"])
    assert np.array_equal(kc.view(np.uint16), z["k_cache"])
    assert np.array_equal(vc.view(np.uint16), z["v_cache"])


def test_norm_rope_decode_fixture():
    z = load("qk_norm_rope_decode.npz")
    hkv = f16(z["k_cache_in"]).shape[0]
    hq = f16(z["q_out"]).shape[0] - hkv
    kc, vc = f16(z["k_cache_in"]).copy(), f16(z["v_cache_in"]).copy()
    qo = np.zeros((hq + hkv, D), np.float16)
    oracle.qk_norm_rope_kv_decode(f16(z["qkv"]), f16(z["q_weight"]), f16(z["k_weight"]),
                                  z["inv_freq"], qo, kc, vc, int(z["position"]),
                                  float(z["eps"]), hq, hkv)
    assert np.array_equal(qo.view(np.uint16), z["q_out"])
    assert np.array_equal(kc.view(np.uint16), z["k_cache"])
    assert np.array_equal(vc.view(np.uint16), z["v_cache"])


def test_attn_prefill_fixture():
    z = load("attn_prefill.npz")
    for key in ("S17_qs0", "S17_qs5", "S64_qs0", "S64_qs5"):
        S, qs = (int(x[1:]) for x in key.replace("qs", "q").split("_"))
        out = oracle.attn_prefill_f32(f16(z[key + "_q"]), f16(z[key + "_k"]), f16(z[key + "_v"]),
                                      1.0 / math.sqrt(D), qs + S, qs)
        assert np.array_equal(out, z[key + "_out"]), key


def test_attn_decode_fixture():
    z = load("attn_decode.npz")
    qg = f16(z["q"])
    for ns in (1, 3):
        att, lse = oracle.attn_decode_split(qg, f16(z["k_cache"]), f16(z["v_cache"]),
                                            int(z["qk_scale_f16"]), int(z["position"]),
                                            int(z["block_n"]), ns)
        assert np.array_equal(att.view(np.uint16), z[f"nks{ns}_att"])
        assert np.array_equal(lse, z[f"nks{ns}_lse"])
        out = oracle.attn_decode_merge(att, lse, qg.shape[1])
        assert np.array_equal(out.view(np.uint16), z[f"nks{ns}_out"])


def test_c1_output_digests():
    """Config c1 end to end through the oracle (norm/RoPE/KV write, then f32
    causal attention) reproduces the committed SHA-256 of every output."""
    import json
    import sys

    sys.path.insert(0, GOLD)
    try:
        import make_golden
    finally:
        sys.path.remove(GOLD)
    with open(os.path.join(GOLD, "c1_sha256.json")) as f:
        want = json.load(f)
    got = make_golden.c1_digests()
    assert got == want
