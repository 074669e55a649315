"""Write the golden fixtures in tests/golden/ from the CPU oracle.

Small shapes (Hq=4, Hkv=2, D=128) with seeded N(0,1) inputs; f16 tensors are
stored as their uint16 bit patterns, f32 as float32, in one .npz per op.
Run from the repository root:  python tests/golden/make_golden.py
"""
import hashlib
import json
import math
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
import oracle  # noqa: E402

OUT = os.path.dirname(os.path.abspath(__file__))
D, EPS, THETA = 128, 1e-6, 1e6
SEED = 0x67726F7574000000


def f16(g, shape):
    return g.standard_normal(shape, dtype=np.float32).astype(np.float16)


def bits(a):
    return np.ascontiguousarray(a).view(np.uint16)


def main():
    g = np.random.default_rng(SEED + 100)
    inv = oracle.build_inv_freq(THETA)
    hq, hkv = 4, 2
    qw = (1 + 0.1 * g.standard_normal(D, dtype=np.float32)).astype(np.float16)
    kw = (1 + 0.1 * g.standard_normal(D, dtype=np.float32)).astype(np.float16)

    # Fused norm/RoPE/KV prefill: S=17 rows at position_start=5 into a 32-slot cache.
    S, ps, MS = 17, 5, 32
    q, k, v = f16(g, (S, hq, D)), f16(g, (S, hkv, D)), f16(g, (S, hkv, D))
    kc = np.zeros((hkv, MS, D), np.float16)
    vc = np.zeros((hkv, MS, D), np.float16)
    qo = oracle.qk_norm_rope_kv_prefill(q, k, v, qw, kw, inv, kc, vc, EPS, ps)
    np.savez_compressed(os.path.join(OUT, "qk_norm_rope_prefill.npz"), q=bits(q), k=bits(k),
                        v=bits(v), q_weight=bits(qw), k_weight=bits(kw), inv_freq=inv,
                        position_start=ps, eps=np.float32(EPS), q_out=bits(qo), k_cache=bits(kc),
                        v_cache=bits(vc))

    # Fused decode variant at position 9 of a 16-slot cache.
    pos, MSd = 9, 16
    qkv = f16(g, ((hq + 2 * hkv) * D,))
    kcd, vcd = f16(g, (hkv, MSd, D)), f16(g, (hkv, MSd, D))
    kc2, vc2 = kcd.copy(), vcd.copy()
    qo2 = np.zeros((hq + hkv, D), np.float16)
    oracle.qk_norm_rope_kv_decode(qkv, qw, kw, inv, qo2, kc2, vc2, pos, EPS, hq, hkv)
    np.savez_compressed(os.path.join(OUT, "qk_norm_rope_decode.npz"), qkv=bits(qkv),
                        q_weight=bits(qw), k_weight=bits(kw), inv_freq=inv, position=pos,
                        eps=np.float32(EPS), k_cache_in=bits(kcd), v_cache_in=bits(vcd),
                        q_out=bits(qo2), k_cache=bits(kc2), v_cache=bits(vc2))

    # Causal prefill attention (fp32 oracle outputs): S in {17, 64}, query_start in {0, 5}.
    cases = {}
    for S_, qs in ((17, 0), (17, 5), (64, 0), (64, 5)):
        MS_ = qs + S_ + 3
        qa = f16(g, (S_, hq, D))
        ka, va = f16(g, (hkv, MS_, D)), f16(g, (hkv, MS_, D))
        out = oracle.attn_prefill_f32(qa, ka, va, 1.0 / math.sqrt(D), qs + S_, qs)
        key = f"S{S_}_qs{qs}"
        cases[key + "_q"] = bits(qa)
        cases[key + "_k"] = bits(ka)
        cases[key + "_v"] = bits(va)
        cases[key + "_out"] = out
    np.savez_compressed(os.path.join(OUT, "attn_prefill.npz"), **cases)

    # Split-K decode + merge: s_kv = 41 (pos 40), BN = 32, NKS in {1, 3}.
    qg = f16(g, (hkv, hq // hkv, D))
    kd, vd = f16(g, (hkv, 48, D)), f16(g, (hkv, 48, D))
    dec = dict(q=bits(qg), k_cache=bits(kd), v_cache=bits(vd), position=40, block_n=32,
               qk_scale_f16=oracle.f16_bits(1.0 / math.sqrt(D)))
    for ns in (1, 3):
        att, lse = oracle.attn_decode_split(qg, kd, vd, dec["qk_scale_f16"], 40, 32, ns)
        dec[f"nks{ns}_att"] = bits(att)
        dec[f"nks{ns}_lse"] = lse
        dec[f"nks{ns}_out"] = bits(oracle.attn_decode_merge(att, lse, hq // hkv))
    np.savez_compressed(os.path.join(OUT, "attn_decode.npz"), **dec)

    # Config c1 (Qwen3-0.6B layer, S=512 at positions 0..511, 16 Q / 8 KV
    # heads, cache of 512 slots): SHA-256 of each oracle output.
    with open(os.path.join(OUT, "c1_sha256.json"), "w") as f:
        json.dump(c1_digests(), f, indent=1, sort_keys=True)
        f.write("\n")
    print("golden fixtures written to", OUT)


C1_SEED = SEED + 1


def c1_digests():
    """Config c1's inputs from C1_SEED (q, k, v ~ N(0,1) f16, norm weights
    1 + N(0, 0.1)), the oracle's fused norm/RoPE/KV write and its f32 causal
    attention on the written cache; SHA-256 of the output bytes (f16 bit
    patterns, f32 little-endian)."""
    g = np.random.default_rng(C1_SEED)
    hq, hkv, S = 16, 8, 512
    q, k, v = f16(g, (S, hq, D)), f16(g, (S, hkv, D)), f16(g, (S, hkv, D))
    qw = (1 + 0.1 * g.standard_normal(D, dtype=np.float32)).astype(np.float16)
    kw = (1 + 0.1 * g.standard_normal(D, dtype=np.float32)).astype(np.float16)
    inv = oracle.build_inv_freq(THETA)
    kc = np.zeros((hkv, S, D), np.float16)
    vc = np.zeros((hkv, S, D), np.float16)
    qo = oracle.qk_norm_rope_kv_prefill(q, k, v, qw, kw, inv, kc, vc, EPS, 0)
    att = oracle.attn_prefill_f32(qo, kc, vc, 1.0 / math.sqrt(D), S, 0)
    sha = lambda a: hashlib.sha256(np.ascontiguousarray(a).tobytes()).hexdigest()  # noqa: E731
    return {"seed": C1_SEED, "shape": {"seq_len": S, "num_q_heads": hq, "num_kv_heads": hkv,
                                       "head_dim": D, "max_seq_len": S},
            "q_out_f16": sha(bits(qo)), "k_cache_f16": sha(bits(kc)),
            "v_cache_f16": sha(bits(vc)), "attn_out_f32": sha(att.astype("<f4"))}


if __name__ == "__main__":
    main()
