"""GPU parity of the split-K prefill (fmha_prefill_gqa_lpt_split +
prefill_splitk_reduce_merge, src/kernels.rs:1872-2323) against the oracle.

Contract: per-split partials within |a-b| <= 2e-3 + 1e-2|b| and LSEs within
1e-3 (log2 units) of oracle.attn_prefill_split wherever the split holds a key
for the row; rows with no key in a split's range carry an LSE below -1e28 on
both sides (weight 0 in the merge).  Merged output within the attention
tolerance of the oracle's merge and of the fp32 full-attention oracle, and,
at the c3 shape, of the unsplit GPU prefill.
"""
import math

import numpy as np
import pytest

import oracle
from tests._util import D, assert_close_attn, normal_f16, rng

pytestmark = pytest.mark.gpu

SCALE = 1.0 / math.sqrt(D)


def _run_split(torch, q, kc, vc, qs, kv_len, bm, bn, gr, ns):
    import grout_amd

    dq = torch.from_numpy(q).cuda()
    dk = torch.from_numpy(kc).cuda()
    dv = torch.from_numpy(vc).cuda()
    S, hq, _ = q.shape
    att, lse = grout_amd.prefill_split_scratch(hq, S, bm, gr, ns)
    att.fill_(float("nan"))  # every scratch row must be written
    grout_amd.attend_prefill_split(dq, dk, dv, att, lse, qs, bm, bn, gr, ns, kv_len=kv_len)
    out = torch.empty_like(dq)
    grout_amd.prefill_splitk_reduce_merge(att, lse, out, bm, gr, ns)
    torch.cuda.synchronize()
    return att.cpu().numpy(), lse.cpu().numpy(), out.cpu().numpy()


@pytest.mark.parametrize("S,qs,kv_len,MS,hq,hkv,bm,bn,gr,ns,seed", [
    (40, 0, 40, 43, 4, 2, 32, 32, 2, 3, 1),       # ragged q_len, padded block rows
    (64, 0, 64, 64, 4, 2, 32, 16, 1, 4, 2),       # GROUP 1, BN below the kernel tile
    (33, 7, 40, 48, 6, 3, 64, 32, 2, 2, 3),       # query_start > 0
    (300, 0, 300, 320, 8, 2, 64, 64, 4, 5, 4),    # G = 4, several q blocks per workgroup
    (130, 0, 130, 160, 64, 8, 32, 32, 8, 3, 5),   # G = 8 (Qwen3-32B heads)
    (200, 100, 300, 300, 12, 4, 96, 48, 3, 7, 6), # G = 3, BM = 96, suffix chunk
    (20, 0, 20, 20, 4, 2, 32, 32, 2, 4, 7),       # splits past tc are empty
])
def test_prefill_split_matches_oracle(gpu, S, qs, kv_len, MS, hq, hkv, bm, bn, gr, ns, seed):
    import torch

    g = rng(40 + seed)
    q = normal_f16(g, (S, hq, D))
    kc, vc = normal_f16(g, (hkv, MS, D)), normal_f16(g, (hkv, MS, D))
    att, lse, out = _run_split(torch, q, kc, vc, qs, kv_len, bm, bn, gr, ns)
    ratt, rlse = oracle.attn_prefill_split(q, kc, vc, SCALE, kv_len, qs, bm, bn, gr, ns)
    assert att.shape == ratt.shape and lse.shape == rlse.shape
    live = rlse > -1e20
    assert live.any()
    assert np.all(lse[~live] < -1e28), "a row without keys in a split must have weight 0"
    assert np.all(att[~live & (rlse == np.float32(-1e30))] == 0), "empty split must store O = 0"
    assert_close_attn(att[live], ratt[live], f"split partials S={S} bm={bm} bn={bn} ns={ns}")
    assert np.max(np.abs(lse[live] - rlse[live])) < 1e-3
    rout = oracle.attn_prefill_split_merge(ratt, rlse, hq, S, bm, gr, ns)
    assert_close_attn(out, rout, "split merge vs oracle merge")
    full = oracle.attn_prefill_f32(q, kc, vc, SCALE, kv_len=kv_len, query_start=qs)
    assert_close_attn(out, full, "split merge vs full attention")


def test_prefill_split_equals_unsplit_at_c3_shape(gpu):
    """c3 shape (S=8192, 32/8 heads): split + merge equals the unsplit kernel."""
    import torch

    import grout_amd

    S, hq, hkv, bm, bn, gr, ns = 8192, 32, 8, 128, 64, 4, 4
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0x67726F7574000003)
    q = torch.randn((S, hq, D), device="cuda", generator=gen).half()
    kc = torch.randn((hkv, S, D), device="cuda", generator=gen).half()
    vc = torch.randn((hkv, S, D), device="cuda", generator=gen).half()
    ref = torch.empty_like(q)
    grout_amd.attend_prefill(q, kc, vc, ref, 0)
    att, lse = grout_amd.prefill_split_scratch(hq, S, bm, gr, ns)
    grout_amd.attend_prefill_split(q, kc, vc, att, lse, 0, bm, bn, gr, ns)
    out = torch.empty_like(q)
    grout_amd.prefill_splitk_reduce_merge(att, lse, out, bm, gr, ns)
    torch.cuda.synchronize()
    assert_close_attn(out.cpu().numpy(), ref.cpu().numpy(), "split vs unsplit at c3")
