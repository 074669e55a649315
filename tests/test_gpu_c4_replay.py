"""Config c4 at its own replay count: the Qwen3-32B decode step (64 Q / 8 KV
heads, context 32768, KV ~ N(0,1)) captured once and replayed 1000x at
positions 32768..33767 with only the position scalar moving between replays
(the replay loop of src/model.rs:2061-2090 and launch_step,
src/model.rs:363-403).

The fused step hands partials between workgroups through relaxed agent-scope
counters and device-coherent stores; this test holds that handoff to the
oracle under sustained replay.  Replays 0, 1, 500 and 999 are checked:
attn_out against the oracle's norm/RoPE/KV write + split + merge at that
position, q_out within 1 f16 ulp, every new K row within 1 ulp and every new V
row bit-exact; at the end the position is 33768 and the counters are zero.
Two further replays at one position must give bit-identical attn_out.
"""
import numpy as np
import pytest

import oracle
from tests._util import (D, EPS, THETA, assert_close_attn, f16_ulp_diff, normal_f16,
                         norm_weight, qk_scale_f16_bits, rng)

pytestmark = pytest.mark.gpu

BN = 32


def test_c4_graph_1000_replays_match_oracle(gpu):
    import torch

    import grout_amd

    g = rng(400)
    hq, hkv, ctx, replays = 64, 8, 32768, 1000
    G = hq // hkv
    MS = ctx + 1024
    kc = np.zeros((hkv, MS, D), np.float16)
    vc = np.zeros((hkv, MS, D), np.float16)
    kc[:, :ctx] = normal_f16(g, (hkv, ctx, D))
    vc[:, :ctx] = normal_f16(g, (hkv, ctx, D))
    qkv = normal_f16(g, ((hq + 2 * hkv) * D,))
    qw, kw = norm_weight(g), norm_weight(g)
    inv = oracle.build_inv_freq(THETA)
    ns = grout_amd.pick_num_splits(MS, hkv)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()  # noqa: E731
    dev = dict(qkv=t(qkv), q_weight=t(qw), k_weight=t(kw), inv_freq=t(inv),
               q_out=torch.zeros(((hq + hkv), D), dtype=torch.float16, device="cuda"),
               k_cache=t(kc), v_cache=t(vc),
               attn_out=torch.zeros((hkv, G, D), dtype=torch.float16, device="cuda"),
               position=torch.zeros((1,), dtype=torch.int32, device="cuda"))
    att, lse = grout_amd.decode_scratch(hkv, G, ns)
    print(f"[c4 replay] 64/8 heads ctx {ctx} NKS {ns}: prime at {ctx}", flush=True)
    runner = grout_amd.DecodeGraphRunner(
        **dev, att_partial=att, lse_partial=lse, eps=EPS, qk_scale_f16_bits=qk_scale_f16_bits(),
        num_q_heads=hq, num_kv_heads=hkv, num_splits=ns, prime_position=ctx)
    # The oracle's caches follow the same writes: every replay stores the rows
    # of the one qkv vector at its position (RoPE differs per position).
    kc_ref, vc_ref = kc.copy(), vc.copy()
    q_rows = {}
    for pos in range(ctx, ctx + replays):
        qo = np.zeros(((hq + hkv), D), np.float16)
        oracle.qk_norm_rope_kv_decode(qkv, qw, kw, inv, qo, kc_ref, vc_ref, pos, EPS, hq, hkv)
        q_rows[pos] = qo
    checks = (0, 1, 500, 999)
    try:
        done = 0
        for r in checks:
            # Replays done .. r issued back to back from C (the graph advances
            # the position between them), then a sync and a check of replay r.
            runner.run(ctx + done, r + 1 - done)
            done = r + 1
            runner.stream.synchronize()
            pos = ctx + r
            print(f"[c4 replay] replay {r} (position {pos})", flush=True)
            assert int(dev["position"].item()) == pos + 1
            qo_dev = dev["q_out"].cpu().numpy()
            assert f16_ulp_diff(qo_dev[:hq], q_rows[pos][:hq]).max() <= 1, f"q_out replay {r}"
            # Attention at `pos` reads slots [0, pos], which the oracle's caches
            # hold as they stand after replay r (later slots are not read).
            qg = np.ascontiguousarray(q_rows[pos][:hq].reshape(hkv, G, D))
            a_ref, l_ref = oracle.attn_decode_split(qg, kc_ref, vc_ref, qk_scale_f16_bits(), pos,
                                                    BN, ns)
            assert_close_attn(dev["attn_out"].cpu().numpy(),
                              oracle.attn_decode_merge(a_ref, l_ref, G), f"attn_out replay {r}")
        assert int(dev["position"].item()) == ctx + replays
        assert int(runner.counters.abs().sum().item()) == 0, "counters not left at zero"
        new_k = dev["k_cache"][:, ctx:ctx + replays].cpu().numpy()
        new_v = dev["v_cache"][:, ctx:ctx + replays].cpu().numpy()
        assert f16_ulp_diff(new_k, kc_ref[:, ctx:ctx + replays]).max() <= 1
        assert np.array_equal(new_v.view(np.uint16), vc_ref[:, ctx:ctx + replays].view(np.uint16))
        # Nothing past the last replay's slot was written.
        assert np.array_equal(dev["k_cache"][:, ctx + replays:].cpu().numpy().view(np.uint16),
                              kc[:, ctx + replays:].view(np.uint16))
        # Two more replays at one position on identical inputs (each rewrites
        # the same row): attn_out is bit-identical, the accumulation order
        # being fixed.
        outs = []
        for _ in range(2):
            runner.run(ctx + 500, 1)
            runner.stream.synchronize()
            outs.append(dev["attn_out"].clone())
        print("[c4 replay] two replays at one position", flush=True)
        assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16)), \
            "attn_out differs between two replays at one position"
    finally:
        runner.close()
