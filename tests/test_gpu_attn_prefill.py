"""GPU parity of the causal flash-attention prefill against the fp32 oracle.

Contract: |gpu - oracle| <= 2e-3 + 1e-2*|oracle| elementwise, oracle =
benchmarks/src/bin/attention_microbench.rs:665-702 generalised to GQA on the cache.
"""
import math

import numpy as np
import pytest

import oracle
from tests._util import D, assert_close_attn, normal_f16, rng

pytestmark = pytest.mark.gpu

SCALE = 1.0 / math.sqrt(D)


def _run(torch, q, kc, vc, qs, kv_len=None):
    import grout_amd

    dq = torch.from_numpy(q).cuda()
    dk = torch.from_numpy(kc).cuda()
    dv = torch.from_numpy(vc).cuda()
    out = torch.empty_like(dq)
    grout_amd.attend_prefill(dq, dk, dv, out, qs, kv_len=kv_len)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def _case(seed, hq, hkv, S, qs, MS, scale_rows=None):
    g = rng(seed)
    q = normal_f16(g, (S, hq, D))
    kc = normal_f16(g, (hkv, MS, D))
    vc = normal_f16(g, (hkv, MS, D))
    if scale_rows is not None:
        idx = g.random((hkv, MS)) < scale_rows
        kc[idx] = (kc[idx].astype(np.float32) * 8).astype(np.float16)
    return q, kc, vc


@pytest.mark.parametrize("hq,hkv,S,qs,MS,seed", [
    (16, 8, 512, 0, 512, 1),      # config c1
    (4, 2, 17, 0, 17, 2),         # tiny, ragged
    (4, 2, 64, 5, 80, 3),         # query_start > 0 on a padded cache
    (8, 8, 100, 0, 128, 4),       # MHA (G = 1), ragged
    (64, 8, 130, 0, 160, 5),      # G = 8 (Qwen3-32B heads)
    (32, 8, 1, 0, 1, 6),          # single row
    (32, 8, 257, 1000, 1400, 7),  # chunked suffix far into the cache
    (12, 4, 200, 0, 200, 8),      # G = 3 (workgroups straddle position tiles)
])
def test_prefill_matches_oracle(gpu, hq, hkv, S, qs, MS, seed):
    import torch

    q, kc, vc = _case(seed, hq, hkv, S, qs, MS)
    out = _run(torch, q, kc, vc, qs)
    ref = oracle.attn_prefill_f32(q, kc, vc, SCALE, kv_len=qs + S, query_start=qs)
    assert_close_attn(out, ref, f"prefill hq={hq} hkv={hkv} S={S} qs={qs}")


def test_prefill_first_row_is_v0(gpu):
    """Row 0 at position 0 sees only key 0: p = 1, l = 1, out = V[kvh, 0] exactly."""
    import torch

    q, kc, vc = _case(40, 8, 2, 96, 0, 96)
    out = _run(torch, q, kc, vc, 0)
    for h in range(8):
        assert np.array_equal(out[0, h].view(np.uint16), vc[h // 4, 0].view(np.uint16))


def test_prefill_outlier_keys(gpu):
    """1% of K rows scaled x8 (config c5's online-softmax stress), S=1024."""
    import torch

    q, kc, vc = _case(41, 64, 8, 1024, 0, 1024, scale_rows=0.01)
    out = _run(torch, q, kc, vc, 0)
    ref = oracle.attn_prefill_f32(q, kc, vc, SCALE, kv_len=1024, query_start=0)
    assert_close_attn(out, ref, "prefill outliers")


def test_chunked_prefill_equals_full(gpu):
    """src/model.rs:6134-6205 invariant: a suffix prefill at query_start>0 over the
    cached prefix equals the same rows of a full prefill."""
    import torch

    q, kc, vc = _case(42, 32, 8, 384, 0, 384)
    full = _run(torch, q, kc, vc, 0)
    cut = 200
    part = _run(torch, np.ascontiguousarray(q[cut:]), kc, vc, cut)
    assert_close_attn(part, full[cut:].astype(np.float32), "chunked vs full", atol=1e-3, rtol=0)


def test_gqa_equals_mha_with_repeated_kv(gpu):
    import torch

    hq, hkv, S = 8, 2, 150
    q, kc, vc = _case(43, hq, hkv, S, 0, S)
    out = _run(torch, q, kc, vc, 0)
    kr = np.ascontiguousarray(np.repeat(kc, hq // hkv, axis=0))
    vr = np.ascontiguousarray(np.repeat(vc, hq // hkv, axis=0))
    out_mha = _run(torch, q, kr, vr, 0)
    assert np.array_equal(out.view(np.uint16), out_mha.view(np.uint16))


@pytest.mark.parametrize("S", [2048])
def test_prefill_long_sampled_rows(gpu, S):
    """Qwen3-4B heads at S=2048; oracle on a stride sample of rows."""
    import torch

    q, kc, vc = _case(44, 32, 8, S, 0, S)
    out = _run(torch, q, kc, vc, 0)
    ref = oracle.attn_prefill_f32(q, kc, vc, SCALE, kv_len=S, query_start=0, row_begin=3,
                                  row_step=61)
    rows = np.arange(3, S, 61)
    assert_close_attn(out[rows], ref[rows], "prefill S=2048 sampled")


@pytest.mark.parametrize("S,G,qs", [(1024, 4, 0), (700, 2, 300)])
def test_small_grid_workgroup_shape_is_bit_identical(gpu, S, G, qs):
    """Grids that fill at most half the CUs run 4-wavefront workgroups, larger
    ones 8-wavefront workgroups; every wavefront computes the same thing in
    both, so a problem and the same problem with more KV heads appended (which
    pushes the grid past the threshold) agree bit for bit on the shared heads."""
    import torch

    cus = torch.cuda.get_device_properties(0).multi_processor_count
    n_pos = -(-S // 32)
    hkv_small = 2
    while 2 * (-(-n_pos * G // 8)) * (hkv_small + 1) <= cus:
        hkv_small += 1
    hkv_big = 2 * hkv_small
    assert 2 * (-(-n_pos * G // 8)) * hkv_small <= cus < 2 * (-(-n_pos * G // 8)) * hkv_big
    print(f"[prefill 4/8 waves] S={S} G={G} Hkv {hkv_small} vs {hkv_big}", flush=True)
    q, kc, vc = _case(400 + S, hkv_big * G, hkv_big, S, qs, qs + S)
    small = _run(torch, np.ascontiguousarray(q[:, :hkv_small * G]), np.ascontiguousarray(kc[:hkv_small]),
                 np.ascontiguousarray(vc[:hkv_small]), qs)
    big = _run(torch, q, kc, vc, qs)
    assert np.array_equal(small.view(np.uint16), big[:, :hkv_small * G].view(np.uint16))
    ref = oracle.attn_prefill_f32(np.ascontiguousarray(q[:, :hkv_small * G]), kc[:hkv_small],
                                  vc[:hkv_small], SCALE, kv_len=qs + S, query_start=qs,
                                  row_step=37)
    assert_close_attn(small[::37], ref[::37], "4-wavefront workgroups, sampled rows")


def _short_form_applies(cus, hq, S, qs, kv_len):
    """The host rule of the short form: every 32-row block needs at most 8 key
    tiles of 64, and one workgroup per (query head, row block) fits the CUs."""
    n_blocks = -(-S // 32)
    return min(kv_len, qs + 32 * n_blocks) <= 8 * 64 and n_blocks * hq <= cus


@pytest.mark.parametrize("hq,hkv,S,qs,MS,kv_len,seed", [
    (16, 8, 50, 40, 96, None, 11),    # rows 40..63's second tile holds none of their keys
    (8, 2, 512, 0, 512, None, 12),    # 8 key tiles in the last row block, G = 4
    (32, 8, 256, 0, 256, None, 13),   # 256 workgroups: one per CU on MI355X
    (4, 1, 300, 200, 512, 480, 14),   # kv_len short of query_start + q_len (rows past it see 480 keys)
    (21, 7, 321, 7, 400, None, 15),   # ragged: a partial last row block, G = 3
    (16, 8, 1, 511, 512, None, 17),   # one row over 512 keys: every wavefront holds a tile
    (8, 4, 32, 480, 512, None, 18),   # one full row block at the end of the range
])
def test_short_prefill_matches_oracle(gpu, hq, hkv, S, qs, MS, kv_len, seed):
    """Launches small enough for the short form (one workgroup per query head
    and 32-row block, one key tile per wavefront, partials merged in LDS)."""
    import torch

    kv = qs + S if kv_len is None else kv_len
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    assert _short_form_applies(cus, hq, S, qs, kv), "shape outside the short form"
    print(f"[short prefill] hq={hq} hkv={hkv} S={S} qs={qs} kv_len={kv}", flush=True)
    q, kc, vc = _case(seed, hq, hkv, S, qs, MS)
    out = _run(torch, q, kc, vc, qs, kv_len=kv)
    ref = oracle.attn_prefill_f32(q, kc, vc, SCALE, kv_len=kv, query_start=qs)
    assert_close_attn(out, ref, f"short prefill hq={hq} hkv={hkv} S={S} qs={qs} kv_len={kv}")


def test_short_prefill_boundary_agrees_with_grid(gpu):
    """The same problem on both sides of the short form's CU rule: the short
    launch and the grid launch (one more query head pushes the grid past one
    workgroup per CU) agree within the attention tolerance on the shared heads."""
    import torch

    cus = torch.cuda.get_device_properties(0).multi_processor_count
    S, G = 256, 2
    hq_short = (cus // (S // 32)) // G * G
    hq_grid = hq_short + G
    assert _short_form_applies(cus, hq_short, S, 0, S) and not _short_form_applies(cus, hq_grid, S, 0, S)
    print(f"[short prefill boundary] hq {hq_short} vs {hq_grid}", flush=True)
    q, kc, vc = _case(16, hq_grid, hq_grid // G, S, 0, S)
    short = _run(torch, np.ascontiguousarray(q[:, :hq_short]), np.ascontiguousarray(kc[:hq_short // G]),
                 np.ascontiguousarray(vc[:hq_short // G]), 0)
    grid = _run(torch, q, kc, vc, 0)
    assert_close_attn(short, grid[:, :hq_short].astype(np.float32), "short vs grid")
    ref = oracle.attn_prefill_f32(q, kc, vc, SCALE, kv_len=S, query_start=0, row_step=13)
    assert_close_attn(grid[::13], ref[::13], "grid, sampled rows")
