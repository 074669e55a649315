"""grout_attn_prefill_sched: the causal prefill with the dynamic per-XCD
schedule (persistent workgroups claiming tasks from queues, heaviest first).

Every task runs the same code as in the static grid, so the output must be
bit-identical to grout_attn_prefill's, which the prefill tests hold to the
oracle (src/kernels.rs:1146-1295); one case also checks sampled rows against
the oracle directly.  The counters must be zero again after every call, and
grids of at most two rounds of workgroups must take the static launch without
touching them.  Shapes cover one KV head per queue (Hkv 8), empty queues that
are drained by stealing from the start (Hkv 4, and Hkv 1 where seven XCDs own
nothing), two heads per queue (Hkv 16), three heads with a ragged last block,
a chunk at query_start > 0, and two calls in a row on one buffer (all of
them grids of more than two rounds of workgroups on 256 CUs).
"""
import math

import numpy as np
import pytest

import oracle
from tests._util import D, assert_close_attn

pytestmark = pytest.mark.gpu


def _inputs(torch, seed, q_len, hq, hkv, ms, outliers=False):
    g = torch.Generator(device="cuda").manual_seed(seed)
    q = torch.randn((q_len, hq, D), device="cuda", generator=g).half()
    kc = torch.randn((hkv, ms, D), device="cuda", generator=g).half()
    vc = torch.randn((hkv, ms, D), device="cuda", generator=g).half()
    if outliers:
        m = torch.rand((hkv, ms), device="cuda", generator=g) < 0.01
        kc[m] = (kc[m].float() * 8).half()
    return q, kc, vc


@pytest.mark.parametrize("q_len,hq,hkv,qs,outliers", [
    (8192, 32, 8, 0, False),     # c3: one KV head per queue
    (6144, 32, 4, 0, True),      # queues 4-7 empty: their workgroups steal from the start
    (4096, 64, 16, 0, False),    # two KV heads per queue, interleaved
    (6144, 32, 8, 1000, False),  # a chunk at query_start > 0
    (20000, 8, 1, 0, False),     # one KV head: seven XCDs steal every heavy and light task
    (12000, 12, 3, 0, True),     # three KV heads, G = 4, ragged last block
    (6144, 24, 12, 0, False),    # twelve KV heads: queues 0-3 hold two heads, 4-7 one
], ids=["c3", "hkv4", "hkv16", "chunk", "hkv1", "hkv3", "hkv12"])
def test_sched_bit_identical_to_static(gpu, q_len, hq, hkv, qs, outliers):
    import torch

    import grout_amd

    print(f"[prefill sched] q_len={q_len} {hq}/{hkv} heads qs={qs}", flush=True)
    q, kc, vc = _inputs(torch, 900 + q_len + hkv, q_len, hq, hkv, qs + q_len, outliers)
    ref = torch.empty_like(q)
    grout_amd.attend_prefill(q, kc, vc, ref, qs)
    counters = grout_amd.prefill_sched_counters()
    out = torch.full_like(q, float("nan"))
    grout_amd.attend_prefill(q, kc, vc, out, qs, sched_counters=counters)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), "sched output differs"
    assert int(counters.abs().sum().item()) == 0, "counters not left at zero"


def test_sched_two_calls_then_oracle_rows(gpu):
    """Two calls in a row on one counter buffer, the second smaller; sampled
    rows of the second against the oracle."""
    import torch

    import grout_amd

    counters = grout_amd.prefill_sched_counters()
    for q_len, seed in ((8192, 910), (6144, 911)):
        q, kc, vc = _inputs(torch, seed, q_len, 32, 8, q_len)
        ref = torch.empty_like(q)
        grout_amd.attend_prefill(q, kc, vc, ref, 0)
        out = torch.empty_like(q)
        grout_amd.attend_prefill(q, kc, vc, out, 0, sched_counters=counters)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), f"q_len={q_len}"
        assert int(counters.abs().sum().item()) == 0
    qn, kn, vn, on = (t.cpu().numpy() for t in (q, kc, vc, out))
    for r in (0, 777, q_len - 1):
        o_ref = oracle.attn_prefill_f32(np.ascontiguousarray(qn[r:r + 1]), kn, vn,
                                        1.0 / math.sqrt(D), kv_len=q_len, query_start=r)[0]
        assert_close_attn(on[r], o_ref, f"sched row {r}")


def test_sched_alternating_inputs_reuse_output(gpu):
    """Stress of the task queues at c3: 40 scheduled launches back to back on one
    counter buffer and one output buffer, alternating between two query inputs.
    A task claimed twice would only rewrite its block, but a task lost or a block
    left unwritten would keep the previous launch's values, from the other input:
    after every launch the whole output must equal the static grid's output for
    that launch's input, bit for bit, and the counters must end at zero."""
    import torch

    import grout_amd

    q_len, hq, hkv, n = 8192, 32, 8, 40
    qa, kc, vc = _inputs(torch, 930, q_len, hq, hkv, q_len)
    qb = _inputs(torch, 931, q_len, hq, hkv, q_len)[0]
    refs = []
    for q in (qa, qb):
        r = torch.empty_like(q)
        grout_amd.attend_prefill(q, kc, vc, r, 0)
        refs.append(r.view(torch.int16))
    counters = grout_amd.prefill_sched_counters()
    out = torch.full_like(qa, float("nan"))
    bad = torch.zeros((n,), dtype=torch.bool, device="cuda")
    print(f"[prefill sched] {n} launches alternating two inputs", flush=True)
    for i in range(n):
        grout_amd.attend_prefill((qa, qb)[i % 2], kc, vc, out, 0, sched_counters=counters)
        bad[i] = (out.view(torch.int16) != refs[i % 2]).any()
    torch.cuda.synchronize()
    assert not bool(bad.any()), f"launches {torch.nonzero(bad).flatten().tolist()[:8]} differ"
    assert not torch.equal(refs[0], refs[1])
    assert int(counters.abs().sum().item()) == 0


def test_small_grid_takes_static_launch(gpu):
    """c1-sized grid (32 workgroups): static launch, counters untouched even
    when they hold a nonzero sentinel."""
    import torch

    import grout_amd

    q, kc, vc = _inputs(torch, 920, 512, 16, 8, 512)
    ref = torch.empty_like(q)
    grout_amd.attend_prefill(q, kc, vc, ref, 0)
    counters = grout_amd.prefill_sched_counters()
    counters.fill_(7)
    out = torch.empty_like(q)
    grout_amd.attend_prefill(q, kc, vc, out, 0, sched_counters=counters)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
    assert bool((counters == 7).all().item()), "static launch touched the counters"
