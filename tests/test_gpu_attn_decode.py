"""GPU parity of split-K GQA decode + merge against the oracle restatement of
src/kernels.rs:2586-2868 and against the fp32 attention oracle."""
import numpy as np
import pytest

import oracle
from tests._util import (D, assert_close_attn, f16_bits_to_f32, normal_f16,
                         qk_scale_f16_bits, rng)

pytestmark = pytest.mark.gpu

BN = 32


def _decode_gpu(torch, qg, kc, vc, pos, ns, bn=BN):
    import grout_amd

    hkv, G, _ = qg.shape
    dq = torch.from_numpy(qg).cuda()
    dk = torch.from_numpy(kc).cuda()
    dv = torch.from_numpy(vc).cuda()
    att, lse = grout_amd.decode_scratch(hkv, G, ns)
    dpos = torch.tensor([pos], dtype=torch.int32, device="cuda")
    grout_amd.fmha_decode_gqa_split(dq, dk, dv, att, lse, qk_scale_f16_bits(), dpos, bn)
    out = torch.empty((hkv, G, D), dtype=torch.float16, device="cuda")
    grout_amd.splitk_reduce_merge(att, lse, out)
    torch.cuda.synchronize()
    return att.cpu().numpy(), lse.cpu().numpy(), out.cpu().numpy()


def _case(seed, hq, hkv, MS):
    g = rng(seed)
    qg = normal_f16(g, (hkv, hq // hkv, D))
    kc = normal_f16(g, (hkv, MS, D))
    vc = normal_f16(g, (hkv, MS, D))
    return qg, kc, vc


def _fp32_decode(qg, kc, vc, pos):
    hkv, G, _ = qg.shape
    q = np.ascontiguousarray(qg.reshape(1, hkv * G, D))
    scale = f16_bits_to_f32(qk_scale_f16_bits())
    out = oracle.attn_prefill_f32(q, kc, vc, scale, kv_len=pos + 1, query_start=pos)
    return out.reshape(hkv, G, D)


@pytest.mark.parametrize("hq,hkv,pos,MS,ns,seed", [
    (32, 8, 4096, 4200, 16, 1),    # config c2 with the reference's NKS=16
    (32, 8, 4096, 4200, 43, 2),    # c2, split count that does not divide the tiles
    (64, 8, 2047, 2048, 64, 3),    # G = 8, cache full to the last slot
    (4, 2, 0, 8, 4, 4),            # s_kv = 1: three empty splits
    (16, 8, 100, 128, 1, 5),       # one split
    (8, 8, 777, 800, 8, 6),        # MHA decode (G = 1)
    (48, 4, 300, 320, 5, 7),       # G = 12
])
def test_split_and_merge_match_oracle(gpu, hq, hkv, pos, MS, ns, seed):
    import torch

    qg, kc, vc = _case(seed, hq, hkv, MS)
    att, lse, out = _decode_gpu(torch, qg, kc, vc, pos, ns)
    att_ref, lse_ref = oracle.attn_decode_split(qg, kc, vc, qk_scale_f16_bits(), pos, BN, ns)
    out_ref = oracle.attn_decode_merge(att_ref, lse_ref, qg.shape[1])

    s_kv = pos + 1
    nonempty = np.array([oracle.decode_split_range(s_kv, BN, ns, s)[0]
                         < oracle.decode_split_range(s_kv, BN, ns, s)[1] for s in range(ns)])
    G = qg.shape[1]
    rows = np.repeat(nonempty, G)
    # Empty splits carry exactly O = 0, LSE = -1e30 (weight 0 in the merge).
    assert np.all(att[:, ~rows] == 0)
    assert np.all(lse[:, ~rows] == np.float32(-1e30))
    assert_close_attn(att[:, rows], att_ref[:, rows], "att_partial")
    assert np.max(np.abs(lse[:, rows] - lse_ref[:, rows])) < 1e-3
    assert_close_attn(out, out_ref, "merged vs oracle merge")
    assert_close_attn(out, _fp32_decode(qg, kc, vc, pos), "merged vs fp32 decode")


def test_split_invariance(gpu):
    """NKS = 1 and NKS = k give the same attention up to f16 partial rounding."""
    import torch

    qg, kc, vc = _case(50, 32, 8, 3000)
    _, _, o1 = _decode_gpu(torch, qg, kc, vc, 2999, 1)
    _, _, o7 = _decode_gpu(torch, qg, kc, vc, 2999, 7)
    _, _, o64 = _decode_gpu(torch, qg, kc, vc, 2999, 64)
    assert_close_attn(o7, o1, "NKS=7 vs 1")
    assert_close_attn(o64, o1, "NKS=64 vs 1")


def test_single_key_returns_v0(gpu):
    import torch

    qg, kc, vc = _case(51, 16, 4, 64)
    _, _, out = _decode_gpu(torch, qg, kc, vc, 0, 3)
    for h in range(4):
        for gg in range(4):
            assert np.array_equal(out[h, gg].view(np.uint16), vc[h, 0].view(np.uint16))


def test_position_clamped_to_cache(gpu):
    """A device position beyond the cache reads no memory outside it: it behaves
    as position max_seq_len-1."""
    import torch

    qg, kc, vc = _case(52, 32, 8, 256)
    _, _, a = _decode_gpu(torch, qg, kc, vc, 255, 8)
    _, _, b = _decode_gpu(torch, qg, kc, vc, 100000, 8)
    assert np.array_equal(a.view(np.uint16), b.view(np.uint16))


def test_decode_equals_prefill_last_row(gpu):
    """A decode at position p equals row p of a causal prefill (same f16-rounded scale)."""
    import torch

    import grout_amd

    hq, hkv, MS, pos = 32, 8, 1100, 1024
    qg, kc, vc = _case(53, hq, hkv, MS)
    _, _, out = _decode_gpu(torch, qg, kc, vc, pos, 16)
    q = torch.from_numpy(np.ascontiguousarray(qg.reshape(1, hq, D))).cuda()
    o2 = torch.empty_like(q)
    grout_amd.attend_prefill(q, torch.from_numpy(kc).cuda(), torch.from_numpy(vc).cuda(), o2,
                             pos, qk_scale=f16_bits_to_f32(qk_scale_f16_bits()))
    torch.cuda.synchronize()
    assert_close_attn(out.reshape(1, hq, D), o2.cpu().numpy().astype(np.float32),
                      "decode vs prefill row")


def test_graph_runner_replay(gpu):
    """DecodeGraphRunner: capture once, replay at successive positions (the graph
    advances the position itself), then jump to a non-consecutive position; each
    replay equals the oracle's norm/RoPE/KV write + split + merge."""
    import torch

    import grout_amd
    from tests._util import EPS, THETA, norm_weight

    g = rng(60)
    hq, hkv, MS, p0 = 32, 8, 640, 500
    G = hq // hkv
    kc = normal_f16(g, (hkv, MS, D))
    vc = normal_f16(g, (hkv, MS, D))
    qw, kw = norm_weight(g), norm_weight(g)
    inv = oracle.build_inv_freq(THETA)
    ns = 12
    dev = dict(
        qkv=torch.zeros(((hq + 2 * hkv) * D,), dtype=torch.float16, device="cuda"),
        q_weight=torch.from_numpy(qw).cuda(), k_weight=torch.from_numpy(kw).cuda(),
        inv_freq=torch.from_numpy(inv).cuda(),
        q_out=torch.zeros(((hq + hkv), D), dtype=torch.float16, device="cuda"),
        k_cache=torch.from_numpy(kc).cuda(), v_cache=torch.from_numpy(vc).cuda(),
        attn_out=torch.zeros((hkv, G, D), dtype=torch.float16, device="cuda"),
        position=torch.zeros((1,), dtype=torch.int32, device="cuda"),
    )
    att, lse = grout_amd.decode_scratch(hkv, G, ns)
    runner = grout_amd.DecodeGraphRunner(
        **dev, att_partial=att, lse_partial=lse, eps=EPS, qk_scale_f16_bits=qk_scale_f16_bits(),
        num_q_heads=hq, num_kv_heads=hkv, num_splits=ns, prime_position=p0)
    kc_ref, vc_ref = kc.copy(), vc.copy()
    try:
        for step, pos in enumerate([p0, p0 + 1, p0 + 2, p0 + 3, p0 + 7, p0 + 8]):
            qkv = normal_f16(g, ((hq + 2 * hkv) * D,))
            with torch.cuda.stream(runner.stream):
                dev["qkv"].copy_(torch.from_numpy(qkv).cuda())
                runner.launch_step(pos)
            runner.stream.synchronize()
            out = dev["attn_out"].cpu().numpy()
            qo_ref = np.zeros(((hq + hkv), D), dtype=np.float16)
            oracle.qk_norm_rope_kv_decode(qkv, qw, kw, inv, qo_ref, kc_ref, vc_ref, pos, EPS,
                                          hq, hkv)
            qg = np.ascontiguousarray(qo_ref[:hq].reshape(hkv, G, D))
            a_ref, l_ref = oracle.attn_decode_split(qg, kc_ref, vc_ref, qk_scale_f16_bits(),
                                                    pos, BN, ns)
            assert_close_attn(out, oracle.attn_decode_merge(a_ref, l_ref, G), f"replay {step}")
        # The prime pass wrote slot p0 once before capture; the replays rewrote it.
        assert int(dev["position"].item()) == p0 + 9
        assert int(runner.counters.abs().sum().item()) == 0
        # run(): four consecutive steps issued from C with one qkv; equals four
        # oracle steps on the same input.
        qkv = normal_f16(g, ((hq + 2 * hkv) * D,))
        with torch.cuda.stream(runner.stream):
            dev["qkv"].copy_(torch.from_numpy(qkv).cuda())
            runner.run(p0 + 20, 4)
        runner.stream.synchronize()
        for pos in range(p0 + 20, p0 + 24):
            qo_ref = np.zeros(((hq + hkv), D), dtype=np.float16)
            oracle.qk_norm_rope_kv_decode(qkv, qw, kw, inv, qo_ref, kc_ref, vc_ref, pos, EPS,
                                          hq, hkv)
        qg = np.ascontiguousarray(qo_ref[:hq].reshape(hkv, G, D))
        a_ref, l_ref = oracle.attn_decode_split(qg, kc_ref, vc_ref, qk_scale_f16_bits(),
                                                p0 + 23, BN, ns)
        assert_close_attn(dev["attn_out"].cpu().numpy(), oracle.attn_decode_merge(a_ref, l_ref, G),
                          "run x4")
        assert int(dev["position"].item()) == p0 + 24
        kc_dev = dev["k_cache"].cpu().numpy()
        from tests._util import f16_ulp_diff
        assert f16_ulp_diff(kc_dev, kc_ref).max() <= 1
        runner.zero_kv_caches()
        assert int(dev["k_cache"].abs().sum().item()) == 0
    finally:
        runner.close()


def _fused_case(seed, hq, hkv, MS):
    from tests._util import norm_weight

    g = rng(seed)
    qkv = normal_f16(g, ((hq + 2 * hkv) * D,))
    qw, kw = norm_weight(g), norm_weight(g)
    kc = normal_f16(g, (hkv, MS, D))
    vc = normal_f16(g, (hkv, MS, D))
    return g, qkv, qw, kw, kc, vc


@pytest.mark.parametrize("hq,hkv,pos,MS,ns,seed", [
    (32, 8, 4096, 4200, 16, 70),   # config c2 shapes
    (32, 8, 4096, 4200, 33, 71),   # split count not dividing the tiles
    (64, 8, 2047, 2048, 32, 72),   # G = 8, last cache slot
    (4, 2, 0, 8, 4, 73),           # s_kv = 1, empty splits
    (16, 16, 300, 512, 3, 74),     # G = 1; 3 LSEs: not whole 16-byte chunks, so the
                                   # merge loads them with the rows (fallback path)
    # The in-kernel merge takes its partial rows in batches of 512 / G splits
    # (one batch at most 64 splits) and carries (max, sum, acc) across them;
    # these need 2-3 batches.
    (32, 4, 4100, 4200, 96, 76),   # G = 8: batches of 64 splits (64 + 32)
    (64, 4, 3000, 3100, 40, 77),   # G = 16: batches of 32 (32 + 8)
    (48, 4, 4000, 4100, 100, 78),  # G = 12: batches of 42 (42 + 42 + 16)
    (8, 1, 3000, 3100, 128, 86),   # one KV head (MQA-style), G = 8: 2 batches of 64 splits
    (64, 8, 131071, 131072, 32, 87),  # 128K context, the last slot: 4096-token splits
    (64, 4, 5000, 5100, 64, 79),   # G = 16: 32 + 32 (4 KV heads' picked split count)
    # One batch, LSE block copied first.
    (64, 8, 3000, 3100, 48, 80),   # G = 8, 48 splits: two weight slots per lane
    (32, 4, 4100, 4200, 64, 84),   # G = 8, 64 splits (4 KV heads' picked split count)
    (64, 4, 5000, 5100, 32, 85),   # G = 16, 32 splits: 512 rows, the grouped picker's count
    (64, 4, 2500, 2600, 16, 81),   # G = 16, 16 splits: two passes of the weight rows
    (32, 8, 3000, 3100, 48, 82),   # G = 4, 48 splits: two weight slots per lane
    # One batch, fallback path (105 LSEs), two weight slots per lane.
    (24, 8, 3000, 3100, 35, 83),   # G = 3
])
def test_fused_step_matches_oracle(gpu, hq, hkv, pos, MS, ns, seed):
    """grout_attn_decode_fused = norm/RoPE/KV write + split + merge of the oracle;
    counters return to zero; the position advances only when asked."""
    import torch

    import grout_amd
    from tests._util import EPS, THETA, f16_ulp_diff

    _, qkv, qw, kw, kc, vc = _fused_case(seed, hq, hkv, MS)
    G = hq // hkv
    inv = oracle.build_inv_freq(THETA)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    dkc, dvc = t(kc), t(vc)
    q_out = torch.full(((hq + hkv), D), 2.5, dtype=torch.float16, device="cuda")
    out = torch.zeros((hkv, G, D), dtype=torch.float16, device="cuda")
    att, lse = grout_amd.decode_scratch(hkv, G, ns)
    counters = grout_amd.decode_counters(hkv)
    dpos = torch.tensor([pos], dtype=torch.int32, device="cuda")
    first = None
    for advance in (False, True):
        grout_amd.decode_fused(t(qkv), t(qw), t(kw), t(inv), q_out, dkc, dvc, att, lse, out,
                               counters, dpos, EPS, qk_scale_f16_bits(), hq, hkv,
                               advance_position=advance)
        torch.cuda.synchronize()
        assert int(dpos.item()) == pos + (1 if advance else 0)
        assert int(counters.abs().sum().item()) == 0, "counters not reset"
        dpos.fill_(pos)
        # Both launches see the same inputs (the second rewrites the same
        # cache row): the accumulation order is fixed, so every output is
        # bit-identical run to run.
        got = [x.clone() for x in (out, att, lse, q_out)]
        if first is None:
            first = got
        else:
            for name, x, y in zip(("attn_out", "att_partial", "lse_partial", "q_out"), first, got):
                assert torch.equal(x.view(torch.int16) if x.dtype == torch.float16 else x.view(torch.int32),
                                   y.view(torch.int16) if y.dtype == torch.float16 else y.view(torch.int32)), \
                    f"{name} differs between two identical launches"

    qo_ref = np.full(((hq + hkv), D), np.float16(2.5), dtype=np.float16)
    kc_ref, vc_ref = kc.copy(), vc.copy()
    oracle.qk_norm_rope_kv_decode(qkv, qw, kw, inv, qo_ref, kc_ref, vc_ref, pos, EPS, hq, hkv)
    qo = q_out.cpu().numpy()
    assert f16_ulp_diff(qo[:hq], qo_ref[:hq]).max() <= 1
    assert np.array_equal(qo[hq:].view(np.uint16), qo_ref[hq:].view(np.uint16))
    kc_dev, vc_dev = dkc.cpu().numpy(), dvc.cpu().numpy()
    assert np.array_equal(vc_dev.view(np.uint16), vc_ref.view(np.uint16))
    assert f16_ulp_diff(kc_dev, kc_ref).max() <= 1
    qg = np.ascontiguousarray(qo_ref[:hq].reshape(hkv, G, D))
    # The fused form's partials stay inside the launch and its splits are
    # balanced 16-token ranges: the partials are held to the oracle's split
    # arithmetic on those ranges, the merged output to the oracle's split +
    # merge on the reference's ranges and to an f32 attention.
    ranges = [oracle.decode_split_range_fused(pos + 1, ns, s) for s in range(ns)]
    a_ref, l_ref = oracle.attn_decode_split(qg, kc_ref, vc_ref, qk_scale_f16_bits(), pos, BN, ns,
                                            fused_ranges=True)
    rows = np.repeat(np.array([b < e for b, e in ranges]), G)
    a_dev, l_dev = att.cpu().numpy(), lse.cpu().numpy()
    assert_close_attn(a_dev[:, rows], a_ref[:, rows], "fused att_partial")
    assert np.max(np.abs(l_dev[:, rows] - l_ref[:, rows])) < 1e-3
    assert np.all(l_dev[:, ~rows] == np.float32(-1e30))
    a_o, l_o = oracle.attn_decode_split(qg, kc_ref, vc_ref, qk_scale_f16_bits(), pos, BN, ns)
    out_ref = oracle.attn_decode_merge(a_o, l_o, G)
    assert_close_attn(out.cpu().numpy(), out_ref, "fused out vs oracle")
    assert_close_attn(out.cpu().numpy(), _fp32_decode(qg, kc_ref, vc_ref, pos),
                      "fused out vs fp32 decode")


def test_fused_consecutive_steps_advance(gpu):
    """Ten launches with advance_position walk the cache forward one slot each,
    with no host write of the position in between."""
    import torch

    import grout_amd
    from tests._util import EPS, THETA

    hq, hkv, MS, p0, ns = 32, 8, 300, 250, 8
    g, _, qw, kw, kc, vc = _fused_case(75, hq, hkv, MS)
    G = hq // hkv
    inv = oracle.build_inv_freq(THETA)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    dkc, dvc, dqw, dkw, dinv = t(kc), t(vc), t(qw), t(kw), t(inv)
    q_out = torch.zeros(((hq + hkv), D), dtype=torch.float16, device="cuda")
    out = torch.zeros((hkv, G, D), dtype=torch.float16, device="cuda")
    att, lse = grout_amd.decode_scratch(hkv, G, ns)
    counters = grout_amd.decode_counters(hkv)
    dpos = torch.tensor([p0], dtype=torch.int32, device="cuda")
    kc_ref, vc_ref = kc.copy(), vc.copy()
    dqkv = torch.empty(((hq + 2 * hkv) * D,), dtype=torch.float16, device="cuda")
    for step in range(10):
        qkv = normal_f16(g, ((hq + 2 * hkv) * D,))
        dqkv.copy_(t(qkv))
        grout_amd.decode_fused(dqkv, dqw, dkw, dinv, q_out, dkc, dvc, att, lse, out, counters,
                               dpos, EPS, qk_scale_f16_bits(), hq, hkv, advance_position=True)
        torch.cuda.synchronize()
        qo_ref = np.zeros(((hq + hkv), D), np.float16)
        oracle.qk_norm_rope_kv_decode(qkv, qw, kw, inv, qo_ref, kc_ref, vc_ref, p0 + step, EPS,
                                      hq, hkv)
        qg = np.ascontiguousarray(qo_ref[:hq].reshape(hkv, G, D))
        a_ref, l_ref = oracle.attn_decode_split(qg, kc_ref, vc_ref, qk_scale_f16_bits(),
                                                p0 + step, BN, ns)
        assert_close_attn(out.cpu().numpy(), oracle.attn_decode_merge(a_ref, l_ref, G),
                          f"step {step}")
    assert int(dpos.item()) == p0 + 10


def test_fused_handoff_alternating_inputs(gpu):
    """Stress of the merge hand-off at the c4 shape (64/8 heads, 32 splits, one
    workgroup per CU): 400 launches at a fixed position alternate between two
    QKV vectors, issued back to back on one stream.  The merger of each head
    reads the partials its head's other workgroups published in the same
    launch; a partial read before its store had landed would be the previous
    launch's, computed from the other input, and would change the output.  So
    every output equals the first output of its input bit for bit, the two
    inputs' outputs differ, and the merge counters end at zero."""
    import torch

    import grout_amd
    from tests._util import EPS, THETA

    hq, hkv, pos, ns, n = 64, 8, 32768, 32, 400
    MS, G = pos + 64, hq // hkv
    gen = torch.Generator(device="cuda").manual_seed(4242)
    dkc = torch.randn((hkv, MS, D), device="cuda", generator=gen).half()
    dvc = torch.randn((hkv, MS, D), device="cuda", generator=gen).half()
    qkvs = [torch.randn(((hq + 2 * hkv) * D,), device="cuda", generator=gen).half()
            for _ in range(2)]
    qw = (1.0 + 0.1 * torch.randn((D,), device="cuda", generator=gen)).half()
    kw = (1.0 + 0.1 * torch.randn((D,), device="cuda", generator=gen)).half()
    inv = torch.from_numpy(oracle.build_inv_freq(THETA)).cuda()
    q_out = torch.zeros(((hq + hkv), D), dtype=torch.float16, device="cuda")
    out = torch.zeros((hkv, G, D), dtype=torch.float16, device="cuda")
    outs = torch.empty((n, hkv, G, D), dtype=torch.float16, device="cuda")
    att, lse = grout_amd.decode_scratch(hkv, G, ns)
    counters = grout_amd.decode_counters(hkv)
    dpos = torch.tensor([pos], dtype=torch.int32, device="cuda")
    print(f"[handoff] {n} fused launches, {hq}/{hkv} heads, {ns} splits", flush=True)
    for i in range(n):
        grout_amd.decode_fused(qkvs[i % 2], qw, kw, inv, q_out, dkc, dvc, att, lse, out, counters,
                               dpos, EPS, qk_scale_f16_bits(), hq, hkv)
        outs[i].copy_(out)
    torch.cuda.synchronize()
    bits = outs.view(torch.int16)
    for k in range(2):
        same = (bits[k::2] == bits[k]).flatten(1).all(dim=1)
        assert bool(same.all()), f"input {k}: launches {torch.nonzero(~same).flatten().tolist()[:8]} differ"
    assert not torch.equal(bits[0], bits[1])
    assert torch.isfinite(outs[:2].float()).all()
    assert int(counters.view(torch.int32).abs().sum().item()) == 0
    assert int(dpos.item()) == pos


def test_fused_position_saturates_past_cache(gpu):
    """A fused step whose device position is at or past max_seq_len writes no
    cache row and, with advance_position, leaves the position where it is; the
    last slot itself (max_seq_len - 1) still advances to max_seq_len."""
    import torch

    import grout_amd
    from tests._util import EPS, THETA

    hq, hkv, MS, ns = 16, 4, 96, 3
    _, qkv, qw, kw, kc, vc = _fused_case(80, hq, hkv, MS)
    G = hq // hkv
    inv = oracle.build_inv_freq(THETA)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    dkc, dvc = t(kc), t(vc)
    q_out = torch.zeros(((hq + hkv), D), dtype=torch.float16, device="cuda")
    out = torch.zeros((hkv, G, D), dtype=torch.float16, device="cuda")
    att, lse = grout_amd.decode_scratch(hkv, G, ns)
    counters = grout_amd.decode_counters(hkv)
    for start, end in ((MS - 1, MS), (MS, MS), (MS + 5, MS + 5)):
        dpos = torch.tensor([start], dtype=torch.int32, device="cuda")
        before_k = dkc.clone()
        grout_amd.decode_fused(t(qkv), t(qw), t(kw), t(inv), q_out, dkc, dvc, att, lse, out,
                               counters, dpos, EPS, qk_scale_f16_bits(), hq, hkv,
                               advance_position=True)
        torch.cuda.synchronize()
        assert int(dpos.item()) == end, f"position {start} -> {int(dpos.item())}"
        assert int(counters.abs().sum().item()) == 0
        if start >= MS:
            assert torch.equal(before_k, dkc), "a position past the cache wrote a K row"


def test_fused_steps_on_two_streams_concurrently(gpu):
    """Two streams, each with its own scratch, counters, position and output,
    run 50 fused decode steps each, interleaved on the host so their launches
    overlap on the GPU (c4 heads, 32 splits: 256 workgroups each, so the two
    grids share the CUs).  Each stream's outputs equal the same steps run
    alone, bit for bit: the kernel keeps no state outside its arguments."""
    import torch

    import grout_amd
    from tests._util import EPS, THETA

    hq, hkv, pos, ns, n = 64, 8, 8192, 32, 50
    MS, G = pos + 64, hq // hkv
    gen = torch.Generator(device="cuda").manual_seed(5151)
    inv = torch.from_numpy(oracle.build_inv_freq(THETA)).cuda()
    qw = (1.0 + 0.1 * torch.randn((D,), device="cuda", generator=gen)).half()
    kw = (1.0 + 0.1 * torch.randn((D,), device="cuda", generator=gen)).half()

    def state():
        kc = torch.randn((hkv, MS, D), device="cuda", generator=gen).half()
        vc = torch.randn((hkv, MS, D), device="cuda", generator=gen).half()
        qkv = torch.randn(((hq + 2 * hkv) * D,), device="cuda", generator=gen).half()
        att, lse = grout_amd.decode_scratch(hkv, G, ns)
        return dict(kc=kc, vc=vc, qkv=qkv, att=att, lse=lse,
                    counters=grout_amd.decode_counters(hkv),
                    q_out=torch.zeros(((hq + hkv), D), dtype=torch.float16, device="cuda"),
                    out=torch.zeros((hkv, G, D), dtype=torch.float16, device="cuda"),
                    outs=torch.empty((n, hkv, G, D), dtype=torch.float16, device="cuda"))

    def launch(s, i):
        grout_amd.decode_fused(s["qkv"], qw, kw, inv, s["q_out"], s["kc"], s["vc"], s["att"],
                               s["lse"], s["out"], s["counters"], s["pos"], EPS,
                               qk_scale_f16_bits(), hq, hkv, advance_position=True)
        s["outs"][i].copy_(s["out"])

    sts = [state(), state()]
    snap = [{k: v.clone() for k, v in s.items()} for s in sts]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    torch.cuda.synchronize()
    print(f"[two streams] {n} fused steps each, interleaved", flush=True)
    for s in sts:
        s["pos"] = torch.tensor([pos], dtype=torch.int32, device="cuda")
    for i in range(n):
        for s, st in zip(sts, streams):
            with torch.cuda.stream(st):
                launch(s, i)
    torch.cuda.synchronize()
    # The same steps, one stream at a time, from the saved starting state.
    for s, ref in zip(sts, snap):
        ref["pos"] = torch.tensor([pos], dtype=torch.int32, device="cuda")
        for i in range(n):
            launch(ref, i)
        torch.cuda.synchronize()
        assert torch.equal(s["outs"].view(torch.int16), ref["outs"].view(torch.int16))
        assert torch.equal(s["kc"].view(torch.int16), ref["kc"].view(torch.int16))
        assert int(s["pos"].item()) == pos + n
        assert int(s["counters"].abs().sum().item()) == 0
