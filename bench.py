#!/usr/bin/env python3
"""Benchmark of the Qwen3 attention hot path on one MI355X.

Headline (BASELINE.json metric): prefill attention TFLOP/s as a fraction of the
fp16 dense MFMA peak, and decode attention GB/s as a fraction of HBM peak.

  value   = config c3: Qwen3-4B causal prefill attention, batch 1, S=8192,
            32 Q / 8 KV heads, head_dim 128, f16 in / f32 accumulate.
            One step = one grout_attn_prefill launch; inputs already in HBM.
  decode  = config c4: Qwen3-32B decode step, 64 Q / 8 KV heads, context
            32768, the fused {norm/RoPE/KV write, split-K decode, merge} step
            captured in a hipGraph and replayed 1000x with only the position
            updated; its roofline is the fused kernel with the KV caches of
            four layers cycled (none resident in the 256 MB last-level cache).
  also    = c1 (Qwen3-0.6B layer, S=512), c2 (Qwen3-4B decode at context
            4096), c5 (Qwen3-32B prefill at S=32768 with 1% outlier keys,
            unsplit and split-K, then 64 graph-replayed decode steps), the
            Qwen3-4B decode at context 32768, c3's fused QK norm/RoPE/KV write
            and KV suffix writer, the decode-layer ops and the whole Qwen3-32B
            and Qwen3-4B token steps.
  steady  = c3 once more at the end, after 200 further untimed launches
            (prefill_c3_steady_state): from idle the GPU's power management
            takes ~50 launches to settle, so the headline window (the
            contract's warmup count) includes that transient.
  power   = board power and per-XCD shader clocks (amd-smi) while c3 and the
            MFMA probe each run for 5 s (power_state).

Kernel durations come from HIP events recorded on the launch stream, around a
run of back-to-back launches divided by the count.  The CPU baseline is the
oracle (a C restatement of the reference's fp32 CPU attention,
benchmarks/src/bin/attention_microbench.rs:665-702) on the host's cores and on
one thread, over stride samples of the same inputs (c5 extrapolated by the
causal work ratio and labelled so).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import itertools
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

# HIP runtime setting for the decode-graph replays, read when HIP initialises
# (main() sets it before torch is imported): with the runtime's graph packet
# capture on (its default), each replay of the one-kernel decode graph costs
# ~4 us more GPU time than the same kernel launched directly; with it off a
# replay costs what a launch costs.  An explicit setting in the environment
# wins; bench.py also measures the c4 graph step under the runtime's default
# in a child process (decode.graph_step_default_runtime_us).
GRAPH_PACKET_ENV = "DEBUG_CLR_GRAPH_PACKET_CAPTURE"

METRIC = ("prefill attn TFLOP/s (% fp16 MFMA peak); decode attn GB/s (% HBM peak), 1 GPU")
PEAK_TFLOPS_F16 = 2516.6   # 256 CU x 4096 FLOP/clk x 2.4 GHz (dense fp16 MFMA)
PEAK_HBM_GBS = 8000.0      # HBM3E
# HBM bytes per launch from rocprofv3 --pmc FETCH_SIZE (x2.0) and WRITE_SIZE (x1.0), the
# scales read off a 1 GiB copy; the runs and figures are in profiles/*.txt.
PMC_TRAFFIC_BYTES = {
    # grout_attn_prefill_sched (the headline's entry point); the static grid read
    # 71776.2 and wrote 65536.0 KiB on the same run.
    "attn_prefill_c3": (74761.5 * 2.0 + 65586.3) * 1024,
    "attn_decode_fused_c4": (65976.8 * 2.0 + 572.3) * 1024,
}
D = 128
EPS = 1e-6
THETA = 1e6


def prefill_flops(hq: int, q_len: int, query_start: int = 0) -> float:
    """2*D*Hq*sum_{m<S}(ps+m+1) x 2 (QK^T and PV MACs, causal incl. diagonal)."""
    pairs = q_len * query_start + q_len * (q_len + 1) // 2
    return 2.0 * 2.0 * D * hq * pairs


def decode_bytes(hq: int, hkv: int, s_kv: int) -> int:
    """K+V read for s_kv keys plus Q in and O out (split scratch not counted)."""
    return 2 * hkv * s_kv * D * 2 + 2 * hq * D * 2


def norm_bytes(hq: int, hkv: int, S: int) -> int:
    """q,k,v read + q_out, k_cache, v_cache rows written."""
    return 2 * S * D * 2 * (hq + 2 * hkv)


def _events(torch, n):
    return [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
            for _ in range(n)]


def time_launches(torch, fn, steps: int, warmup: int, stream=None):
    """Per-launch durations (ms) from event pairs on the launch stream, plus the
    wall time of the whole timed region (ms) between two synchronizations."""
    s = stream or torch.cuda.current_stream()
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    evs = _events(torch, steps)
    t0 = time.perf_counter()
    for a, b in evs:
        a.record(s)
        fn()
        b.record(s)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3
    durs = [a.elapsed_time(b) for a, b in evs]
    return durs, wall


def time_region(torch, fn, steps: int, warmup: int, stream=None):
    """The timed region of the bench contract: `warmup` untimed launches, a
    synchronization, then exactly `steps` launches back to back between two
    events on the launch stream and a synchronization.  Returns the average
    duration per launch (ms, from the events) and the host wall time of the
    region (ms)."""
    s = stream or torch.cuda.current_stream()
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    a.record(s)
    for _ in range(steps):
        fn()
    b.record(s)
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) * 1e3
    return a.elapsed_time(b) / steps, wall


def time_back_to_back(torch, fn, n: int, warmup: int, stream=None) -> float:
    """Average duration (ms) of n launches issued back to back between two events."""
    s = stream or torch.cuda.current_stream()
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record(s)
    for _ in range(n):
        fn()
    b.record(s)
    torch.cuda.synchronize()
    return a.elapsed_time(b) / n


def time_graph_cycle(torch, fn, per_graph: int, launches: int, stream) -> float:
    """Average duration (ms) of one launch of fn, from events around replays of a
    hipGraph that holds `per_graph` consecutive calls of fn (about `launches`
    launches in all): launches back to back on the device without the host's
    per-launch cost, which is longer than a short kernel such as c2's decode
    step (issued from Python, c2's step measured ~1.5 us longer than its kernel
    trace).  fn must not synchronize (it is captured)."""
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for _ in range(per_graph):
            fn()
    replays = max(3, -(-launches // per_graph))
    with torch.cuda.stream(stream):
        for _ in range(2):
            g.replay()
        torch.cuda.synchronize()
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(replays):
            g.replay()
        b.record(stream)
        torch.cuda.synchronize()
    del g
    return a.elapsed_time(b) / (replays * per_graph)


def bench_prefill(torch, ga, steps, warmup, gen):
    hq, hkv, S = 32, 8, 8192
    q = torch.randn((S, hq, D), device="cuda", generator=gen, dtype=torch.float32).half()
    kc = torch.randn((hkv, S, D), device="cuda", generator=gen, dtype=torch.float32).half()
    vc = torch.randn((hkv, S, D), device="cuda", generator=gen, dtype=torch.float32).half()
    out = torch.empty_like(q)
    counters = ga.prefill_sched_counters()
    fn = lambda: ga.attend_prefill(q, kc, vc, out, 0, sched_counters=counters)  # noqa: E731
    ms, wall = time_region(torch, fn, steps, warmup)
    assert torch.isfinite(out).all().item(), "non-finite prefill output"
    # The static grid (grout_attn_prefill) right after, same inputs: its output
    # is bit-identical, only the schedule differs.
    out_st = torch.empty_like(q)
    sfn = lambda: ga.attend_prefill(q, kc, vc, out_st, 0)  # noqa: E731
    static_ms, _ = time_region(torch, sfn, steps, 2)
    assert torch.equal(out_st.view(torch.int16), out.view(torch.int16)), "schedules disagree"
    del out_st
    flops = prefill_flops(hq, S)
    tflops = flops / (ms * 1e-3) / 1e12
    return dict(q=q, kc=kc, vc=vc, out=out, ms=ms, wall_ms=wall, tflops=tflops, flops=flops,
                hq=hq, hkv=hkv, S=S, static_ms=static_ms, counters=counters)


def bench_prefill_steady(torch, ga, pre, steps, sustain=200):
    """The c3 prefill once the GPU's power management has settled: `sustain`
    untimed launches on the c3 inputs, then `steps` launches timed as in
    time_region.  From idle the first ~50 launches run slower (launches 5-25
    average ~560 us against ~490 us after ~60 launches on the same box), so a
    short warmup measures that transient rather than the kernel."""
    fn = lambda: ga.attend_prefill(pre["q"], pre["kc"], pre["vc"], pre["out"], 0,  # noqa: E731
                                   sched_counters=pre["counters"])
    ms, _ = time_region(torch, fn, steps, sustain)
    return dict(ms=ms, tflops=pre["flops"] / (ms * 1e-3) / 1e12, sustain=sustain)


AMD_SMI = "/opt/rocm/bin/amd-smi"


def _smi_sample():
    """(socket power W, [gfx clock MHz per XCD]) from one `amd-smi metric` query,
    or None when the tool is missing or its output is not understood."""
    import subprocess

    try:
        r = subprocess.run([AMD_SMI, "metric", "-p", "-c", "--json"], capture_output=True,
                           text=True, timeout=20)
        g = json.loads(r.stdout)["gpu_data"][0]
        clocks = g["clock"]
        gfx = [clocks[k]["clk"]["value"] for k in sorted(clocks) if k.startswith("gfx_")]
        return float(g["power"]["socket_power"]["value"]), [float(x) for x in gfx]
    except Exception:  # noqa: BLE001 - telemetry is optional
        return None


def bench_power_state(torch, ga, pre, seconds: float = 5.0):
    """Board power and per-XCD shader clocks while the c3 prefill runs back to
    back for `seconds`, then while the MFMA ceiling probe does, sampled with
    amd-smi from a second thread (the readings refresh about once a second, so
    only samples from the second half of each phase count).  Shows whether a
    phase runs at the power limit and at which clock; the fp16 dense peak at
    the measured mean clock is 256 CU x 4096 FLOP/clk x clock.  Returns None
    when amd-smi is unavailable."""
    import threading

    if not os.path.exists(AMD_SMI) or _smi_sample() is None:
        return None
    samples, stop = [], threading.Event()

    def sampler():
        while not stop.is_set():
            s = _smi_sample()
            if s is not None:
                samples.append((time.time(), s))
            stop.wait(0.2)

    th = threading.Thread(target=sampler, daemon=True)
    th.start()

    def phase(fn, per_call):
        torch.cuda.synchronize()
        t0 = time.time()
        rates = []
        while time.time() - t0 < seconds:
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record()
            r = fn()
            b.record()
            b.synchronize()
            rates.append((time.time(), r if r is not None else a.elapsed_time(b) / per_call))
        t1 = time.time()
        mid = t0 + 0.5 * (t1 - t0)
        ss = [s for t, s in samples if mid <= t <= t1]
        late = sorted(r for t, r in rates if t >= mid)
        if not ss or not late:
            return None
        pw = sorted(p for p, _ in ss)
        nx = len(ss[0][1])
        clk = [sorted(c[i] for _, c in ss)[len(ss) // 2] for i in range(nx)]
        return {"socket_power_w": pw[len(pw) // 2], "gfx_clock_mhz": clk,
                "samples": len(ss), "median_rate": late[len(late) // 2]}

    n = 20

    def prefill_chunk():
        for _ in range(n):
            ga.attend_prefill(pre["q"], pre["kc"], pre["vc"], pre["out"], 0,
                              sched_counters=pre["counters"])

    try:
        pf = phase(prefill_chunk, n)
        pr = phase(lambda: bench_mfma_probe(torch, launches=8)["mix"], 1)
        time.sleep(2.0)
        idle = [s for t, s in samples if t >= time.time() - 1.0]
    finally:
        stop.set()
        th.join()

    def at_clock(clk):
        return 256 * 4096 * (sum(clk) / len(clk)) * 1e6 / 1e12

    out = {"seconds_per_phase": seconds, "tool": "amd-smi metric -p -c"}
    if pf is not None:
        ms = pf.pop("median_rate")
        tf = pre["flops"] / (ms * 1e-3) / 1e12
        pk = at_clock(pf["gfx_clock_mhz"])
        pf.update({"ms_per_launch": round(ms, 4), "TFLOP/s": round(tf, 1),
                   "fp16_dense_peak_at_clock": round(pk, 1), "frac_of_peak_at_clock": round(tf / pk, 4)})
        out["prefill_c3"] = pf
    if pr is not None:
        mix = pr.pop("median_rate")
        pk = at_clock(pr["gfx_clock_mhz"])
        pr.update({"mix_TFLOP/s": round(mix, 1), "fp16_dense_peak_at_clock": round(pk, 1),
                   "frac_of_peak_at_clock": round(mix / pk, 4)})
        out["mfma_probe"] = pr
    if idle:
        out["after_2s_idle"] = {"socket_power_w": idle[-1][0], "gfx_clock_mhz": idle[-1][1]}
    return out


def bench_prefill_split(torch, ga, pre, steps, num_splits=4, block_m=128, block_n=64):
    """Split-K prefill (fmha_prefill_gqa_lpt_split + merge) on the c3 inputs of
    bench_prefill: per-launch event times of the split kernel and of the merge."""
    q, kc, vc = pre["q"], pre["kc"], pre["vc"]
    S, hq, hkv = pre["S"], pre["hq"], pre["hkv"]
    gr = hq // hkv
    att, lse = ga.prefill_split_scratch(hq, S, block_m, gr, num_splits)
    out = torch.empty_like(q)
    fn = lambda: ga.attend_prefill_split(q, kc, vc, att, lse, 0, block_m, block_n, gr,  # noqa
                                         num_splits)
    durs, _ = time_launches(torch, fn, steps, 5)
    mfn = lambda: ga.prefill_splitk_reduce_merge(att, lse, out, block_m, gr, num_splits)  # noqa
    mdurs, _ = time_launches(torch, mfn, steps, 5)
    diff = (out.float() - pre["out"].float()).abs().max().item()
    ms, mms = sum(durs) / len(durs), sum(mdurs) / len(mdurs)
    return dict(ms=ms, merge_ms=mms, tflops=pre["flops"] / ((ms + mms) * 1e-3) / 1e12,
                max_diff_vs_unsplit=diff, num_splits=num_splits, block_m=block_m,
                block_n=block_n, group=gr)


def bench_norm(torch, ga, steps, warmup, gen):
    """qk_norm_rope_kv_prefill at c3 shapes (201.3 MB per launch), launches issued from
    a captured graph (no host cost between them).  `ms`: one set of buffers, which the
    256 MB last-level cache partly serves between launches.  `cold_ms`: launches
    cycling over four sets (805 MB), so every launch streams its inputs and outputs
    from and to HBM."""
    hq, hkv, S = 32, 8, 8192
    qw = (1 + 0.1 * torch.randn((D,), device="cuda", generator=gen)).half()
    kw = (1 + 0.1 * torch.randn((D,), device="cuda", generator=gen)).half()
    inv = ga.build_inv_freq(THETA).cuda()
    sets = []
    for _ in range(4):
        q = torch.randn((S, hq, D), device="cuda", generator=gen).half()
        k = torch.randn((S, hkv, D), device="cuda", generator=gen).half()
        v = torch.randn((S, hkv, D), device="cuda", generator=gen).half()
        kc = torch.zeros((hkv, S, D), device="cuda", dtype=torch.float16)
        sets.append((q, k, v, torch.empty_like(q), kc, torch.zeros_like(kc)))
    q, k, v, out, kc, vc = sets[0]
    ga.qk_norm_rope_kv_prefill(q, k, v, qw, kw, inv, out, kc, vc, EPS, 0)  # mirror checks once
    # Through the C entry point, like the other short kernels' legs.
    L = ga.lib()
    gs = torch.cuda.Stream()
    calls = [(q.data_ptr(), k.data_ptr(), v.data_ptr(), qw.data_ptr(), kw.data_ptr(),
              inv.data_ptr(), o.data_ptr(), c.data_ptr(), w.data_ptr(), EPS, 0, S, hq, hkv, D,
              S, gs.cuda_stream) for q, k, v, o, c, w in sets]
    torch.cuda.synchronize()
    fn = lambda: L.grout_qk_norm_rope_kv_prefill(*calls[0])  # noqa: E731
    ms = time_graph_cycle(torch, fn, 12, max(steps, 60), gs)
    it = itertools.cycle(calls)
    cfn = lambda: L.grout_qk_norm_rope_kv_prefill(*next(it))  # noqa: E731
    cold_ms = time_graph_cycle(torch, cfn, 12, max(steps, 60), gs)  # 3 passes over the 4 sets
    nb = norm_bytes(hq, hkv, S)
    return dict(ms=ms, bytes=nb, gbs=nb / (ms * 1e-3) / 1e9, cold_ms=cold_ms,
                cold_gbs=nb / (cold_ms * 1e-3) / 1e9)


def bench_kv_update(torch, ga, steps, warmup, gen):
    """kv_cache_update_seq at c3 shapes: 8192 rows x 8 KV heads of K and V into
    a [8, 8192, 128] cache (read 33.6 MB, write 33.6 MB), launches issued from a
    captured graph (the ~10 us kernel is close to the host's per-launch cost).
    `ms`: one set of buffers (last-level cache resident); `cold_ms`: cycling over
    ten sets (671 MB; 336 MB of inputs, as the non-temporal cache stores do not stay
    in the 256 MB last-level cache), every launch from and to HBM."""
    hkv, S = 8, 8192
    sets = []
    for _ in range(10):
        nk = torch.randn((S, hkv, D), device="cuda", generator=gen).half()
        nv = torch.randn((S, hkv, D), device="cuda", generator=gen).half()
        kc = torch.zeros((hkv, S, D), device="cuda", dtype=torch.float16)
        sets.append((nk, nv, kc, torch.zeros_like(kc)))
    ga.kv_cache_update_seq(*sets[0], 0)  # argument checks of the Python mirror once
    L = ga.lib()
    gs = torch.cuda.Stream()
    calls = [(nk.data_ptr(), nv.data_ptr(), kc.data_ptr(), vc.data_ptr(), 0, S, hkv, D, S,
              gs.cuda_stream) for nk, nv, kc, vc in sets]
    torch.cuda.synchronize()
    fn = lambda: L.grout_kv_cache_update_seq(*calls[0])  # noqa: E731
    ms = time_graph_cycle(torch, fn, 20, max(steps, 100), gs)
    it = itertools.cycle(calls)
    cfn = lambda: L.grout_kv_cache_update_seq(*next(it))  # noqa: E731
    cold_ms = time_graph_cycle(torch, cfn, 20, max(steps, 100), gs)  # 2 passes over the 10 sets
    nb = 2 * 2 * S * hkv * D * 2
    return dict(ms=ms, bytes=nb, gbs=nb / (ms * 1e-3) / 1e9, cold_ms=cold_ms,
                cold_gbs=nb / (cold_ms * 1e-3) / 1e9)


def bench_decode(torch, ga, hq, hkv, ctx, replays, warmup, gen, split_steps, graph_only=False,
                 cold_caches=4):
    """Graph replay of {norm/RoPE/KV write, split, merge} at positions ctx..ctx+replays-1,
    plus event-timed eager launches of the split kernel alone at position ctx.  The
    caches-cycled figures rotate through `cold_caches` layers' caches, enough that no
    launch finds its K/V in the 256 MB last-level cache."""
    G = hq // hkv
    MS = ctx + max(replays, 1024)
    kc = torch.randn((hkv, MS, D), device="cuda", generator=gen).half()
    vc = torch.randn((hkv, MS, D), device="cuda", generator=gen).half()
    qkv = torch.randn(((hq + 2 * hkv) * D,), device="cuda", generator=gen).half()
    qw = (1 + 0.1 * torch.randn((D,), device="cuda", generator=gen)).half()
    kw = (1 + 0.1 * torch.randn((D,), device="cuda", generator=gen)).half()
    inv = ga.build_inv_freq(THETA).cuda()
    q_out = torch.zeros(((hq + hkv), D), device="cuda", dtype=torch.float16)
    attn_out = torch.zeros((hkv, G, D), device="cuda", dtype=torch.float16)
    pos_t = torch.zeros((1,), device="cuda", dtype=torch.int32)
    ns = ga.pick_num_splits(MS, hkv)
    att, lse = ga.decode_scratch(hkv, G, ns)
    scale_bits = f16_scale_bits(torch)
    runner = ga.DecodeGraphRunner(
        qkv=qkv, q_weight=qw, k_weight=kw, inv_freq=inv, q_out=q_out, k_cache=kc, v_cache=vc,
        att_partial=att, lse_partial=lse, attn_out=attn_out, position=pos_t, eps=EPS,
        qk_scale_f16_bits=scale_bits, num_q_heads=hq, num_kv_heads=hkv, num_splits=ns,
        prime_position=ctx)
    s = runner.stream
    try:
        for i in range(warmup):
            runner.launch_step(ctx + i % replays)
        torch.cuda.synchronize()
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(s)
        runner.run(ctx, replays)  # replays issued from C, one graph launch per step
        b.record(s)
        torch.cuda.synchronize()
        step_us = a.elapsed_time(b) * 1e3 / replays
        assert torch.isfinite(attn_out).all().item(), "non-finite decode output"
    finally:
        runner.close()
    # Bytes of the average replayed step (s_kv grows by one per replay).
    avg_bytes = sum(decode_bytes(hq, hkv, ctx + i + 1) for i in range(replays)) / replays
    if graph_only:
        return dict(step_us=step_us, step_gbs=avg_bytes / (step_us * 1e-6) / 1e9,
                    replays=replays)

    # The fused step alone (the graph's only kernel) at position ctx (s_kv =
    # ctx + 1, position not advanced), launched back to back from a captured
    # graph; then the standalone split and merge ops of the same shape.
    counters = ga.decode_counters(hkv)
    pos_t.fill_(ctx)
    with torch.cuda.stream(s):
        ffn = lambda: ga.decode_fused(qkv, qw, kw, inv, q_out, kc, vc, att, lse, attn_out,  # noqa
                                      counters, pos_t, EPS, scale_bits, hq, hkv)
        fused_us = 1e3 * time_graph_cycle(torch, ffn, 16, split_steps, s)
        q_grouped = q_out[:hq].view(hkv, G, D)
        fn = lambda: ga.fmha_decode_gqa_split(q_grouped, kc, vc, att, lse, scale_bits, pos_t)  # noqa
        split_us = 1e3 * time_graph_cycle(torch, fn, 16, split_steps, s)
        # The same fused step cycling through several layers' caches, so no
        # launch finds its K/V in the 256 MB last-level cache: the situation of
        # a real token step, where the other layers run between two reads of
        # one layer's cache.
        nc = cold_caches
        kcs = [kc] + [torch.randn_like(kc) for _ in range(nc - 1)]
        vcs = [vc] + [torch.randn_like(vc) for _ in range(nc - 1)]
        it = [0]

        def cold():
            it[0] += 1
            c = it[0] % nc
            ga.decode_fused(qkv, qw, kw, inv, q_out, kcs[c], vcs[c], att, lse, attn_out,
                            counters, pos_t, EPS, scale_bits, hq, hkv)
        cold_us = 1e3 * time_graph_cycle(torch, cold, 4 * nc, split_steps, s)

        def split_cold():
            it[0] += 1
            c = it[0] % nc
            ga.fmha_decode_gqa_split(q_grouped, kcs[c], vcs[c], att, lse, scale_bits, pos_t)
        split_cold_us = 1e3 * time_graph_cycle(torch, split_cold, 4 * nc, split_steps, s)
        del kcs, vcs
        mfn = lambda: ga.splitk_reduce_merge(att, lse, attn_out)  # noqa: E731
        # A ~4 us kernel launched back to back through the Python mirror is
        # host-bound; per-launch event pairs bound it from above instead.
        mdurs, _ = time_launches(torch, mfn, split_steps, 10, stream=s)
        merge_us = 1e3 * sum(mdurs) / len(mdurs)
    bytes_step = decode_bytes(hq, hkv, ctx + 1)
    return dict(
        hq=hq, hkv=hkv, ctx=ctx, num_splits=ns, replays=replays, step_us=step_us,
        step_gbs=avg_bytes / (step_us * 1e-6) / 1e9, fused_us=fused_us, cold_us=cold_us,
        split_cold_us=split_cold_us,
        cold_gbs=bytes_step / (cold_us * 1e-6) / 1e9,
        fused_gbs=bytes_step / (fused_us * 1e-6) / 1e9, split_us=split_us, merge_us=merge_us,
        split_gbs=bytes_step / (split_us * 1e-6) / 1e9, bytes_step=bytes_step,
        kc=kc, vc=vc, q=q_out[:hq].clone())


def gemv_bytes(m: int, k: int) -> int:
    """Weight [m, k] and x [k] read once, out [m] written (f16)."""
    return 2 * (m * k + k + m)


def bench_decode_layer(torch, ga, steps, gen):
    """The decode-layer ops of the c4 model (Qwen3-32B: hidden 5120, 64 Q / 8 KV
    heads, vocab 151936) through the C entry points, back to back.  Each GEMV
    cycles through enough weight copies (>= 600 MB) that no launch finds its
    weight in the 256 MB last-level cache, as in a real token step where 64
    layers' weights pass between two reads of one matrix."""
    L = ga.lib()
    st = torch.cuda.current_stream().cuda_stream
    res = {}
    for name, m, k in (("qkv_proj", 10240, 5120), ("o_proj", 5120, 8192),
                       ("lm_head", 151936, 5120)):
        copies = max(1, -(-600_000_000 // (2 * m * k)))
        ws = [(torch.randn((m, k), device="cuda", generator=gen) * (k ** -0.5)).half()
              for _ in range(copies)]
        x = torch.randn((k,), device="cuda", generator=gen).half()
        out = torch.empty((m,), device="cuda", dtype=torch.float16)
        ga.gemv_f16(ws[0], x, out)  # argument checks of the Python mirror once
        ptrs = [w.data_ptr() for w in ws]
        it = [0]

        def fn():
            it[0] += 1
            return L.grout_gemv_f16(ptrs[it[0] % copies], x.data_ptr(), out.data_ptr(), m, k, st)

        n = max(steps, 60) if m * k < 1 << 28 else max(steps, 20)
        ms = time_back_to_back(torch, fn, n, 2 * copies)
        nb = gemv_bytes(m, k)
        res[name] = dict(m=m, k=k, us=ms * 1e3, gbs=nb / (ms * 1e-3) / 1e9, bytes=nb,
                         weight_copies=copies)
        del ws
    n = 5120
    r = torch.randn((n,), device="cuda", generator=gen).half()
    x = torch.randn((n,), device="cuda", generator=gen).half()
    w = (1 + 0.1 * torch.randn((n,), device="cuda", generator=gen)).half()
    o = torch.empty_like(r)
    ro = torch.empty_like(r)
    # The two short kernels run back to back from a captured graph (the stream
    # is looked up at each call: the capture stream).
    cur = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731
    args = (r.data_ptr(), x.data_ptr(), w.data_ptr(), o.data_ptr(), ro.data_ptr(), EPS, n)
    gs = torch.cuda.Stream()
    res["add_rms_norm"] = dict(n=n, us=1e3 * time_graph_cycle(
        torch, lambda: L.grout_add_rms_norm_decode(*args, cur()), 50, max(steps, 200), gs))
    v = 151936
    lg = torch.randn((v,), device="cuda", generator=gen).half()
    bm, bi = ga.argmax_scratch(v)
    tok = torch.empty((1,), device="cuda", dtype=torch.int32)
    aargs = (lg.data_ptr(), bm.data_ptr(), bi.data_ptr(), tok.data_ptr(), v)
    res["argmax"] = dict(n=v, us=1e3 * time_graph_cycle(
        torch, lambda: L.grout_argmax_f16(*aargs, cur()), 50, max(steps, 200), gs))
    assert int(tok.item()) == int(torch.argmax(lg.float()).item()), "argmax mismatch"
    return res


# (layers, hidden, intermediate, Q heads, KV heads) of the token-step legs.
QWEN3_32B = (64, 5120, 25600, 64, 8)
QWEN3_4B = (36, 2560, 9728, 32, 8)


def bench_token_step(torch, ga, gen, model=QWEN3_32B, ctx=32768, steps=20):
    """The whole Qwen3 decode token step (`model` = layers, hidden, intermediate,
    Q / KV heads; vocab 151936) as one hipGraph, every layer's KV cache holding
    `ctx` tokens: `steps` replays issued back to back from C, each embedding the
    token the previous one picked.  Random f16 weights; bytes per token = every
    weight matrix + the KV read and written."""
    layers, hidden, inter, hq, hkv = model
    vocab = 151936
    MS = ctx + 1024
    dev = "cuda"

    def mat(m, k, scale=1.0):
        return torch.empty((m, k), dtype=torch.float16, device=dev).normal_(
            0.0, scale / math.sqrt(k), generator=gen)

    def nw(n):
        return torch.empty((n,), dtype=torch.float16, device=dev).normal_(1.0, 0.1, generator=gen)

    def cache():
        return torch.empty((hkv, MS, D), dtype=torch.float16, device=dev).normal_(generator=gen)

    lay = [dict(input_norm=nw(hidden), qkv_proj=mat((hq + 2 * hkv) * D, hidden), q_norm=nw(D),
                k_norm=nw(D), o_proj=mat(hidden, hq * D), post_attn_norm=nw(hidden),
                gate_up_proj=mat(2 * inter, hidden), down_proj=mat(hidden, inter),
                k_cache=cache(), v_cache=cache()) for _ in range(layers)]
    embed = torch.empty((vocab, hidden), dtype=torch.float16, device=dev).normal_(generator=gen)
    lm_head = mat(vocab, hidden, 4.0)
    token = torch.tensor([1], dtype=torch.int32, device=dev)
    position = torch.zeros((1,), dtype=torch.int32, device=dev)
    logits = torch.empty((vocab,), dtype=torch.float16, device=dev)
    scale_bits = int(torch.tensor([1.0 / math.sqrt(D)], dtype=torch.float16).view(torch.int16)
                     .item()) & 0xFFFF
    runner = ga.Qwen3DecodeRunner(
        layers=lay, embed_tokens=embed, final_norm=nw(hidden), lm_head=lm_head,
        inv_freq=ga.build_inv_freq(THETA).cuda(), token=token, position=position, logits=logits,
        num_q_heads=hq, num_kv_heads=hkv, eps=EPS, qk_scale_f16_bits=scale_bits,
        prime_position=ctx)
    s = runner.stream
    try:
        runner.run(ctx + 1, 3)
        torch.cuda.synchronize()
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(s)
        runner.run(ctx + 4, steps)
        b.record(s)
        torch.cuda.synchronize()
        ms = a.elapsed_time(b) / steps
        assert torch.isfinite(logits).all().item(), "non-finite logits"
        assert int(position.item()) == ctx + 4 + steps
    finally:
        runner.close()
    w_layer = 2 * hidden * ((hq + 2 * hkv) * D + hq * D + 3 * inter)
    avg_ctx = ctx + 4 + (steps + 1) / 2
    kv_layer = 2 * hkv * avg_ctx * D * 2 + 2 * hkv * D * 2
    nbytes = layers * (w_layer + kv_layer) + 2 * vocab * hidden + 2 * hidden
    del lay, embed, lm_head
    torch.cuda.empty_cache()
    return dict(ms=ms, tokens_per_s=1e3 / ms, bytes=nbytes, gbs=nbytes / (ms * 1e-3) / 1e9,
                layers=layers, ctx=ctx, steps=steps, num_splits=runner.num_splits)


def bench_mfma_probe(torch, launches: int = 8):
    """Sustained v_mfma_f32_32x32x16_f16 rate for operand data distributed like the
    prefill kernel's (bench_probes/mfma_ceiling.hip), operands loaded once from
    16 MB f16 buffers: A ~ N(0,1) with B ~ N(0,1) (the Q K^T kind) or B = u1*u2 in
    [0,1) (the P V kind).  Returns TFLOP/s per kind and the rate of an equal mix of
    the two (harmonic mean: equal MFMA counts)."""
    import ctypes

    import bench_probes

    lib = ctypes.CDLL(bench_probes.lib_path())
    fn = lib.grout_probe_mfma_f16
    fn.restype = ctypes.c_int32
    fn.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int32,
                   ctypes.c_int32, ctypes.c_void_p]
    blocks = torch.cuda.get_device_properties(0).multi_processor_count
    iters = 4000
    n_chunks = 1 << 20
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0x67726F7574000009)
    a_ops = torch.randn((n_chunks * 8,), device="cuda", generator=gen).half()
    b_kinds = {"qk": torch.randn((n_chunks * 8,), device="cuda", generator=gen).half(),
               "pv": (torch.rand((n_chunks * 8,), device="cuda", generator=gen) *
                      torch.rand((n_chunks * 8,), device="cuda", generator=gen)).half()}
    out = torch.empty((blocks * 512,), device="cuda", dtype=torch.float32)
    stream = torch.cuda.current_stream()
    res = {}
    for kind, b_ops in b_kinds.items():
        call = lambda: fn(a_ops.data_ptr(), b_ops.data_ptr(), n_chunks, out.data_ptr(), blocks, iters,
                          stream.cuda_stream)
        for _ in range(3):
            assert call() == 0
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(launches):
            assert call() == 0
        b.record(stream)
        torch.cuda.synchronize()
        flops = launches * blocks * 8.0 * iters * 16 * 32768
        res[kind] = flops / (a.elapsed_time(b) * 1e-3) / 1e12
    mix = 2.0 / (1.0 / res["qk"] + 1.0 / res["pv"])
    del a_ops, b_kinds
    return dict(qk=res["qk"], pv=res["pv"], mix=mix, blocks=blocks)


def bench_hbm_probe(torch, gib: int = 4, launches: int = 5):
    """Sustained HBM read rate of a plain streaming kernel (bench_probes/hbm_read.hip)
    over a buffer far larger than the 256 MB last-level cache, the best of 1, 2 and 4
    workgroups per CU: the practical ceiling of the HBM-bound kernels.  GB/s (1e9
    bytes)."""
    import ctypes

    import bench_probes

    lib = ctypes.CDLL(bench_probes.lib_path())
    fn = lib.grout_probe_hbm_read
    fn.restype = ctypes.c_int32
    fn.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int32, ctypes.c_void_p]
    nbytes = gib << 30
    src = torch.empty((nbytes,), dtype=torch.uint8, device="cuda").fill_(1)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    out = torch.empty((4 * cus * 256,), dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream()
    best = None
    for per_cu in (1, 2, 4):
        blocks = per_cu * cus
        for _ in range(2):
            assert fn(src.data_ptr(), nbytes, out.data_ptr(), blocks, stream.cuda_stream) == 0
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(launches):
            assert fn(src.data_ptr(), nbytes, out.data_ptr(), blocks, stream.cuda_stream) == 0
        b.record(stream)
        torch.cuda.synchronize()
        gbs = launches * nbytes / (a.elapsed_time(b) * 1e-3) / 1e9
        if best is None or gbs > best["gbs"]:
            best = dict(gbs=gbs, bytes=nbytes, blocks=blocks, workgroups_per_cu=per_cu)
    del src
    torch.cuda.empty_cache()
    return best


def bench_hbm_copy_probe(torch, gib: int = 2, launches: int = 5):
    """Sustained rate of a plain streaming copy (bench_probes/hbm_copy.hip), bytes read
    plus bytes written, over buffers far larger than the 256 MB last-level cache; the
    best of 4 and 8 workgroups per CU.  The practical ceiling of kernels that read and
    write HBM in equal parts (the QK norm/RoPE/KV write, the KV-cache suffix writer).
    GB/s (1e9 bytes)."""
    import ctypes

    import bench_probes

    lib = ctypes.CDLL(bench_probes.lib_path())
    fn = lib.grout_probe_hbm_copy
    fn.restype = ctypes.c_int32
    fn.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_void_p]
    nbytes = gib << 30
    src = torch.empty((nbytes,), dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.zeros((nbytes,), dtype=torch.uint8, device="cuda")
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    stream = torch.cuda.current_stream()
    best = None
    for per_cu in (4, 8):
        blocks = per_cu * cus
        for _ in range(2):
            assert fn(src.data_ptr(), dst.data_ptr(), nbytes, blocks, stream.cuda_stream) == 0
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(launches):
            assert fn(src.data_ptr(), dst.data_ptr(), nbytes, blocks, stream.cuda_stream) == 0
        b.record(stream)
        torch.cuda.synchronize()
        gbs = launches * 2 * nbytes / (a.elapsed_time(b) * 1e-3) / 1e9
        if best is None or gbs > best["gbs"]:
            best = dict(gbs=gbs, bytes=2 * nbytes, blocks=blocks, workgroups_per_cu=per_cu)
    assert bool(torch.equal(src[: 1 << 20], dst[: 1 << 20])), "copy probe wrote wrong bytes"
    del src, dst
    torch.cuda.empty_cache()
    return best


def bench_prefill_c1(torch, ga, gen, n: int = 200):
    """c1: Qwen3-0.6B layer, S=512, 16 Q / 8 KV heads: the fused QK norm/RoPE/KV
    write, then causal prefill attention on the cache it wrote.  Both kernels
    are a few microseconds, so each is timed over n launches back to back from
    a captured graph (no host cost between them)."""
    hq, hkv, S = 16, 8, 512
    q = torch.randn((S, hq, D), device="cuda", generator=gen).half()
    k = torch.randn((S, hkv, D), device="cuda", generator=gen).half()
    v = torch.randn((S, hkv, D), device="cuda", generator=gen).half()
    qw = (1 + 0.1 * torch.randn((D,), device="cuda", generator=gen)).half()
    kw = (1 + 0.1 * torch.randn((D,), device="cuda", generator=gen)).half()
    inv = ga.build_inv_freq(THETA).cuda()
    kc = torch.zeros((hkv, S, D), device="cuda", dtype=torch.float16)
    vc = torch.zeros_like(kc)
    qo = torch.empty_like(q)
    out = torch.empty_like(q)
    ga.qk_norm_rope_kv_prefill(q, k, v, qw, kw, inv, qo, kc, vc, EPS, 0)
    ga.attend_prefill(qo, kc, vc, out, 0)
    L = ga.lib()
    cur = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731
    nargs = (q.data_ptr(), k.data_ptr(), v.data_ptr(), qw.data_ptr(), kw.data_ptr(),
             inv.data_ptr(), qo.data_ptr(), kc.data_ptr(), vc.data_ptr(), EPS, 0, S, hq, hkv, D,
             S)
    pargs = (qo.data_ptr(), kc.data_ptr(), vc.data_ptr(), out.data_ptr(), 1.0 / math.sqrt(D),
             hq, hkv, D, S, S, 0, S)
    gs = torch.cuda.Stream()
    norm_ms = time_graph_cycle(torch, lambda: L.grout_qk_norm_rope_kv_prefill(*nargs, cur()), 50, n, gs)
    attn_ms = time_graph_cycle(torch, lambda: L.grout_attn_prefill(*pargs, cur()), 50, n, gs)
    assert torch.isfinite(out).all().item(), "non-finite c1 output"
    flops = prefill_flops(hq, S)
    nb = norm_bytes(hq, hkv, S)
    return dict(attn_us=attn_ms * 1e3, tflops=flops / (attn_ms * 1e-3) / 1e12, flops=flops,
                norm_us=norm_ms * 1e3, norm_gbs=nb / (norm_ms * 1e-3) / 1e9, norm_bytes=nb,
                q=qo, kc=kc, vc=vc, hq=hq, hkv=hkv, S=S)


def make_c5_inputs(torch, gen, hq=64, hkv=8, S=32768, extra=64):
    """c5: Q/K/V ~ N(0,1) taken as post-norm/RoPE attention inputs, cache
    [8, S + extra, 128]; 1% of the K rows of [0, S) scaled by 8 to stress the
    online-softmax rescale."""
    MS = S + extra
    q = torch.randn((S, hq, D), device="cuda", generator=gen).half()
    kc = torch.zeros((hkv, MS, D), device="cuda", dtype=torch.float16)
    vc = torch.zeros_like(kc)
    kc[:, :S].normal_(generator=gen)
    vc[:, :S].normal_(generator=gen)
    outlier = torch.rand((hkv, S), device="cuda", generator=gen) < 0.01
    kc[:, :S][outlier] *= 8
    return dict(q=q, kc=kc, vc=vc, hq=hq, hkv=hkv, S=S, MS=MS,
                n_outlier_rows=int(outlier.sum().item()))


def bench_c5(torch, ga, gen, steps: int = 5, warmup: int = 3, decode_steps: int = 64,
             split=(2, 256, 64)):
    """c5: Qwen3-32B causal prefill, S=32768, 64 Q / 8 KV heads, 1% of K rows x8;
    the unsplit kernel and the split-K form (N3: NKS, BM, BN = `split`) on the
    same inputs; then `decode_steps` graph-replayed decode steps appending to
    the same cache (fused norm/RoPE/KV write + split-K + merge)."""
    c5 = make_c5_inputs(torch, gen)
    q, kc, vc, hq, hkv, S = c5["q"], c5["kc"], c5["vc"], c5["hq"], c5["hkv"], c5["S"]
    out = torch.empty_like(q)
    counters = ga.prefill_sched_counters()
    fn = lambda: ga.attend_prefill(q, kc, vc, out, 0, sched_counters=counters)  # noqa: E731
    ms, _ = time_region(torch, fn, steps, warmup)
    assert torch.isfinite(out).all().item(), "non-finite c5 prefill output"
    out_st = torch.empty_like(q)
    static_ms, _ = time_region(torch, lambda: ga.attend_prefill(q, kc, vc, out_st, 0), steps, 1)
    assert torch.equal(out_st.view(torch.int16), out.view(torch.int16)), "c5 schedules disagree"
    del out_st
    flops = prefill_flops(hq, S)
    # Split-K prefill (fmha_prefill_gqa_lpt_split + merge) on the same inputs.
    ns, bm, bn = split
    gr = hq // hkv
    att, lse = ga.prefill_split_scratch(hq, S, bm, gr, ns)
    out_s = torch.empty_like(q)
    sfn = lambda: ga.attend_prefill_split(q, kc, vc, att, lse, 0, bm, bn, gr, ns)  # noqa: E731
    mfn = lambda: ga.prefill_splitk_reduce_merge(att, lse, out_s, bm, gr, ns)  # noqa: E731
    split_ms, _ = time_region(torch, sfn, steps, 2)
    merge_ms, _ = time_region(torch, mfn, steps, 2)
    split_diff = (out_s.float() - out.float()).abs().max().item()
    del att, lse, out_s
    torch.cuda.empty_cache()

    # 64 decode steps at positions S .. S+63 through the graph runner.
    G = hq // hkv
    qkv = torch.randn(((hq + 2 * hkv) * D,), device="cuda", generator=gen).half()
    qw = (1 + 0.1 * torch.randn((D,), device="cuda", generator=gen)).half()
    kw = (1 + 0.1 * torch.randn((D,), device="cuda", generator=gen)).half()
    inv = ga.build_inv_freq(THETA).cuda()
    q_out = torch.zeros(((hq + hkv), D), device="cuda", dtype=torch.float16)
    attn_out = torch.zeros((hkv, G, D), device="cuda", dtype=torch.float16)
    pos_t = torch.zeros((1,), device="cuda", dtype=torch.int32)
    dns = ga.pick_num_splits(c5["MS"], hkv)
    datt, dlse = ga.decode_scratch(hkv, G, dns)
    runner = ga.DecodeGraphRunner(
        qkv=qkv, q_weight=qw, k_weight=kw, inv_freq=inv, q_out=q_out, k_cache=kc, v_cache=vc,
        att_partial=datt, lse_partial=dlse, attn_out=attn_out, position=pos_t, eps=EPS,
        qk_scale_f16_bits=f16_scale_bits(torch), num_q_heads=hq, num_kv_heads=hkv,
        num_splits=dns, prime_position=S)
    s = runner.stream
    try:
        torch.cuda.synchronize()
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(s)
        runner.run(S, decode_steps)
        b.record(s)
        torch.cuda.synchronize()
        dec_us = a.elapsed_time(b) * 1e3 / decode_steps
        assert int(pos_t.item()) == S + decode_steps
        assert torch.isfinite(attn_out).all().item(), "non-finite c5 decode output"
    finally:
        runner.close()
    dec_bytes = sum(decode_bytes(hq, hkv, S + i + 1) for i in range(decode_steps))
    return dict(ms=ms, tflops=flops / (ms * 1e-3) / 1e12, flops=flops, static_ms=static_ms,
                split_ms=split_ms,
                merge_ms=merge_ms, split_tflops=flops / ((split_ms + merge_ms) * 1e-3) / 1e12,
                split=split, split_max_diff=split_diff, decode_steps=decode_steps,
                decode_us=dec_us, decode_bytes=dec_bytes,
                decode_gbs=dec_bytes / decode_steps / (dec_us * 1e-6) / 1e9, decode_splits=dns,
                n_outlier_rows=c5["n_outlier_rows"], inputs=c5)


def f16_scale_bits(torch) -> int:
    """f16::from_f32(1/sqrt(128)) (src/model.rs:3427)."""
    return int(torch.tensor([1.0 / math.sqrt(D)], dtype=torch.float16).view(torch.int16)
               .item()) & 0xFFFF


def bench_decode_layers_graph(torch, ga, gen, hq, hkv, ctx, layers, replays):
    """The fused decode step of `layers` layers (one KV cache each, together
    larger than the 256 MB last-level cache) captured in one hipGraph, as in a
    real token step where the other layers' caches pass between two reads of
    one layer's: per-layer step time = replay time / layers.  Only the last
    layer advances the position.  Returns microseconds per layer step."""
    import ctypes

    G = hq // hkv
    MS = ctx + replays + 8
    L = ga.lib()
    caches = [(torch.empty((hkv, MS, D), device="cuda", dtype=torch.float16).normal_(generator=gen),
               torch.empty((hkv, MS, D), device="cuda", dtype=torch.float16).normal_(generator=gen))
              for _ in range(layers)]
    qkv = torch.randn(((hq + 2 * hkv) * D,), device="cuda", generator=gen).half()
    qw = (1 + 0.1 * torch.randn((D,), device="cuda", generator=gen)).half()
    kw = (1 + 0.1 * torch.randn((D,), device="cuda", generator=gen)).half()
    inv = ga.build_inv_freq(THETA).cuda()
    q_out = torch.zeros(((hq + hkv), D), device="cuda", dtype=torch.float16)
    attn_out = torch.zeros((hkv, G, D), device="cuda", dtype=torch.float16)
    pos_t = torch.full((1,), ctx, device="cuda", dtype=torch.int32)
    ns = ga.pick_num_splits(MS, hkv)
    att, lse = ga.decode_scratch(hkv, G, ns)
    counters = ga.decode_counters(hkv)
    stream = torch.cuda.Stream()
    sb = f16_scale_bits(torch)

    def record():
        for i, (kc, vc) in enumerate(caches):
            st = L.grout_attn_decode_fused(
                qkv.data_ptr(), qw.data_ptr(), kw.data_ptr(), inv.data_ptr(), q_out.data_ptr(),
                kc.data_ptr(), vc.data_ptr(), att.data_ptr(), lse.data_ptr(), attn_out.data_ptr(),
                counters.data_ptr(), pos_t.data_ptr(), EPS, sb, hq, hkv, D, MS, 32, ns,
                1 if i == layers - 1 else 0, stream.cuda_stream)
            assert st == 0, f"decode_fused status {st}"

    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        record()  # eager prime pass: errors surface outside capture
    stream.synchronize()
    graph = ctypes.c_void_p()
    assert L.grout_graph_begin(stream.cuda_stream) == 0
    record()
    assert L.grout_graph_end(stream.cuda_stream, ctypes.byref(graph)) == 0
    try:
        for _ in range(3):
            assert L.grout_graph_launch(graph, stream.cuda_stream) == 0
        stream.synchronize()
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record(stream)
        for _ in range(replays):
            assert L.grout_graph_launch(graph, stream.cuda_stream) == 0
        b.record(stream)
        stream.synchronize()
        us = a.elapsed_time(b) * 1e3 / (replays * layers)
        assert int(pos_t.item()) == ctx + 1 + 3 + replays
    finally:
        L.grout_graph_destroy(graph)
    del caches
    torch.cuda.empty_cache()
    avg_bytes = decode_bytes(hq, hkv, ctx + 4 + (replays + 1) // 2)
    return dict(us=us, gbs=avg_bytes / (us * 1e-6) / 1e9, layers=layers, replays=replays,
                num_splits=ns)


def host_threads():
    """(threads used, host CPUs visible): all CPUs this process may run on,
    capped by OMP_NUM_THREADS when it is set (the CPU share of a shared box)."""
    visible = len(os.sched_getaffinity(0))
    cap = os.environ.get("OMP_NUM_THREADS")
    threads = min(visible, int(cap)) if cap and cap.isdigit() and int(cap) > 0 else visible
    return threads, visible


def _cpu_prefill_rate(q, kc, vc, S, hq, query_start, kv_len, row_step, threads):
    """The oracle's fp32 attention (cpu_reference restated) over query rows
    0::row_step, all heads; returns (TFLOP/s, seconds, rows)."""
    import oracle

    t0 = time.perf_counter()
    oracle.attn_prefill_f32(q, kc, vc, 1.0 / math.sqrt(D), kv_len, query_start, row_begin=0,
                            row_step=row_step, nthreads=threads)
    dt = time.perf_counter() - t0
    rows = range(0, S, row_step)
    flops = sum(2.0 * 2.0 * D * hq * (query_start + m + 1) for m in rows)
    return flops / dt / 1e12, dt, len(rows)


def cpu_baselines(torch, pre, dec, c5, c1):
    """The reference's CPU attention path (a C restatement of cpu_reference,
    benchmarks/src/bin/attention_microbench.rs:665-702: fp32, two-pass softmax,
    generalised to GQA on the cache and to decode) on this host, at all the
    threads this process may use and at 1 thread, on bounded samples of the
    configs' own inputs."""
    import oracle

    threads, visible = host_threads()
    res = {"threads": threads, "host_cpus_visible": visible}
    # c3 prefill: every row on all threads; rows 0::32 on one.
    q = pre["q"].cpu().numpy()
    kc = pre["kc"].cpu().numpy()
    vc = pre["vc"].cpu().numpy()
    S, hq = pre["S"], pre["hq"]
    r_all, t_all, n_all = _cpu_prefill_rate(q, kc, vc, S, hq, 0, S, 1, threads)
    r_one, t_one, n_one = _cpu_prefill_rate(q, kc, vc, S, hq, 0, S, 32, 1)
    res["c3"] = dict(value=r_all, unit="TFLOP/s", cores=threads, single_thread_value=r_one,
                     sample=f"c3 in full: all {n_all} query rows x {hq} heads on {threads} "
                            f"threads ({t_all:.1f} s); rows 0::32 ({n_one} of {S}) on 1 "
                            f"thread ({t_one:.1f} s)")
    del q, kc, vc
    # c1 in full (norm output as the attention input), all threads and 1.
    q1 = c1["q"].cpu().numpy()
    k1 = c1["kc"].cpu().numpy()
    v1 = c1["vc"].cpu().numpy()
    r1, t1, _ = _cpu_prefill_rate(q1, k1, v1, c1["S"], c1["hq"], 0, c1["S"], 1, threads)
    r1s, t1s, _ = _cpu_prefill_rate(q1, k1, v1, c1["S"], c1["hq"], 0, c1["S"], 1, 1)
    res["c1"] = dict(value=r1, unit="TFLOP/s", cores=threads, single_thread_value=r1s,
                     sample=f"c1 in full: {t1 * 1e3:.0f} ms on {threads} threads, "
                            f"{t1s * 1e3:.0f} ms on 1")

    # Decode steps: one c4 step (s_kv = ctx + 1) on all threads and on one.
    def decode_rate(d, nthreads):
        hq_, hkv_, ctx = d["hq"], d["hkv"], d["ctx"]
        qd = d["q"].cpu().numpy().reshape(1, hq_, D)
        kd = d["kc"][:, :ctx + 1].contiguous().cpu().numpy()
        vd = d["vc"][:, :ctx + 1].contiguous().cpu().numpy()
        t0 = time.perf_counter()
        oracle.attn_prefill_f32(qd, kd, vd, 0.08837890625, ctx + 1, ctx, nthreads=nthreads)
        dt = time.perf_counter() - t0
        return decode_bytes(hq_, hkv_, ctx + 1) / dt / 1e9, dt

    g_all, dt_all = decode_rate(dec, threads)
    g_one, dt_one = decode_rate(dec, 1)
    res["c4"] = dict(value=g_all, unit="GB/s", cores=threads, single_thread_value=g_one,
                     sample=f"one c4 decode step (s_kv={dec['ctx'] + 1}, {dec['hq']} heads): "
                            f"{dt_all * 1e3:.0f} ms on {threads} threads, {dt_one * 1e3:.0f} ms "
                            "on 1")
    # c5 prefill: rows 0::256 of all heads, extrapolated to the whole config by
    # the exact causal work ratio; then its 64 decode steps in full.
    inp = c5["inputs"]
    q5 = inp["q"].cpu().numpy()
    k5 = inp["kc"].cpu().numpy()
    v5 = inp["vc"].cpu().numpy()
    S5, hq5 = inp["S"], inp["hq"]
    r5, t5, n5 = _cpu_prefill_rate(q5, k5, v5, S5, hq5, 0, S5, 256, threads)
    full_s = c5["flops"] / (r5 * 1e12)
    del q5
    res["c5"] = dict(value=r5, unit="TFLOP/s", cores=threads, extrapolated=True,
                     extrapolated_full_prefill_s=full_s,
                     sample=f"c5 inputs, query rows 0::256 ({n5} of {S5}) x {hq5} heads on "
                            f"{threads} threads ({t5:.1f} s), extrapolated to all rows by the "
                            "causal work ratio")
    qd = torch.randn((1, hq5, D), generator=torch.Generator().manual_seed(5)).half().numpy()
    t0 = time.perf_counter()
    for i in range(c5["decode_steps"]):
        oracle.attn_prefill_f32(qd, k5, v5, 0.08837890625, S5 + i + 1, S5 + i, nthreads=threads)
    dt = time.perf_counter() - t0
    res["c5_decode"] = dict(value=c5["decode_bytes"] / dt / 1e9, unit="GB/s", cores=threads,
                            sample=f"c5's {c5['decode_steps']} decode steps in full "
                                   f"(s_kv {S5 + 1}..{S5 + c5['decode_steps']}): {dt:.1f} s on "
                                   f"{threads} threads")
    return res


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__,
                                 formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    # 50 warmup launches (~30 ms of prefill) bring the clocks up from idle;
    # with 5 the first timed launches still run ramping up.
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--decode-replays", type=int, default=1000)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only", choices=["all", "prefill", "prefill-split", "decode", "norm", "kv",
                                       "mfma-probe", "decode-layer", "token-step", "hbm-probe",
                                       "c1", "c5", "decode-graph-step", "power"],
                    default="all",
                    help="run one workload only (for profiling runs); prints no JSON line "
                         "(decode-graph-step prints the c4 graph step as one JSON line)")
    ap.add_argument("--hip-default-graph-capture", action="store_true",
                    help=f"leave {GRAPH_PACKET_ENV} unset (the HIP runtime's default)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run a plain 1 GiB device-to-device copy (reads and writes 1 GiB) "
                         "to scale rocprofv3 FETCH_SIZE/WRITE_SIZE readings, then exit")
    args = ap.parse_args(argv)
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(attention would shard by KV head with no communication, each GPU "
              "running these kernels on its heads' share).",
              file=sys.stderr)
        return 2
    if not args.hip_default_graph_capture:
        os.environ.setdefault(GRAPH_PACKET_ENV, "0")
    packet_capture = os.environ.get(GRAPH_PACKET_ENV, "runtime default")

    import torch

    import grout_amd as ga

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 2
    ga.lib()
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0x67726F7574000003)

    def log(msg):
        print(f"[bench] {msg}", file=sys.stderr, flush=True)

    if args.copy_calibration:
        src = torch.empty((1 << 30,), dtype=torch.uint8, device="cuda").fill_(1)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log("copy calibration: 3 x 1 GiB device copies done")
        return 0
    if args.only != "all":
        if args.only == "prefill":
            pre = bench_prefill(torch, ga, args.steps, args.warmup, gen)
            log(f"prefill c3: {pre['ms']:.3f} ms/launch, {pre['tflops']:.1f} TFLOP/s (static grid {pre['static_ms']:.3f} ms)")
        elif args.only == "norm":
            nrm = bench_norm(torch, ga, args.steps, args.warmup, gen)
            log(f"norm c3: {nrm['ms'] * 1e3:.1f} us, {nrm['gbs']:.0f} GB/s; cycled "
                f"{nrm['cold_ms'] * 1e3:.1f} us, {nrm['cold_gbs']:.0f} GB/s")
        elif args.only == "kv":
            kvu = bench_kv_update(torch, ga, args.steps, args.warmup, gen)
            log(f"kv update c3: {kvu['ms'] * 1e3:.1f} us, {kvu['gbs']:.0f} GB/s; cycled "
                f"{kvu['cold_ms'] * 1e3:.1f} us, {kvu['cold_gbs']:.0f} GB/s")
        elif args.only == "prefill-split":
            pre = bench_prefill(torch, ga, args.steps, args.warmup, gen)
            psp = bench_prefill_split(torch, ga, pre, args.steps)
            log(f"prefill c3: {pre['ms'] * 1e3:.1f} us; split-K: split {psp['ms'] * 1e3:.1f} us + "
                f"merge {psp['merge_ms'] * 1e3:.1f} us, max |split - unsplit| "
                f"{psp['max_diff_vs_unsplit']:.2e}")
        elif args.only == "decode-layer":
            dl = bench_decode_layer(torch, ga, args.steps, gen)
            log("decode layer c4: " + ", ".join(
                f"{k} {v['us']:.2f} us" + (f" ({v['gbs']:.0f} GB/s)" if "gbs" in v else "")
                for k, v in dl.items()))
        elif args.only == "token-step":
            ts = bench_token_step(torch, ga, gen, steps=args.steps)
            log(f"token step c4 ({ts['layers']} layers, ctx {ts['ctx']}): {ts['ms']:.3f} ms/token, "
                f"{ts['tokens_per_s']:.1f} tok/s, {ts['gbs']:.0f} GB/s")
            t4 = bench_token_step(torch, ga, gen, model=QWEN3_4B, steps=args.steps)
            log(f"token step Qwen3-4B ({t4['layers']} layers, ctx {t4['ctx']}): "
                f"{t4['ms']:.3f} ms/token, {t4['tokens_per_s']:.1f} tok/s, {t4['gbs']:.0f} GB/s")
        elif args.only == "hbm-probe":
            hp = bench_hbm_probe(torch)
            log(f"hbm read probe: {hp['gbs']:.0f} GB/s over {hp['bytes'] >> 30} GiB "
                f"({hp['workgroups_per_cu']} workgroups per CU)")
            cp = bench_hbm_copy_probe(torch)
            log(f"hbm copy probe: {cp['gbs']:.0f} GB/s read + write "
                f"({cp['workgroups_per_cu']} workgroups per CU)")
        elif args.only == "mfma-probe":
            mp = bench_mfma_probe(torch)
            log(f"mfma probe: QK operands {mp['qk']:.0f}, PV operands {mp['pv']:.0f}, "
                f"mix {mp['mix']:.0f} TFLOP/s")
        elif args.only == "c1":
            c1 = bench_prefill_c1(torch, ga, gen)
            log(f"c1: attention {c1['attn_us']:.2f} us ({c1['tflops']:.1f} TFLOP/s), norm "
                f"{c1['norm_us']:.2f} us ({c1['norm_gbs']:.0f} GB/s)")
        elif args.only == "c5":
            c5 = bench_c5(torch, ga, gen, steps=args.steps, warmup=min(args.warmup, 5))
            log(f"c5: prefill {c5['ms']:.2f} ms ({c5['tflops']:.1f} TFLOP/s); split-K "
                f"{c5['split_ms']:.2f} + {c5['merge_ms']:.2f} ms; decode {c5['decode_us']:.2f} "
                f"us/step")
        elif args.only == "power":
            pre = bench_prefill(torch, ga, args.steps, args.warmup, gen)
            pw = bench_power_state(torch, ga, pre)
            log(f"power state: {json.dumps(pw)}")
        elif args.only == "decode-graph-step":
            dec = bench_decode(torch, ga, 64, 8, 32768, args.decode_replays, 20, gen, 200,
                               graph_only=True)
            print(json.dumps({"graph_step_us": round(dec["step_us"], 3),
                              "graph_step_gbs": round(dec["step_gbs"], 1),
                              "replays": dec["replays"], "packet_capture": packet_capture}),
                  flush=True)
        else:
            dec = bench_decode(torch, ga, 64, 8, 32768, args.decode_replays, args.warmup, gen,
                               args.steps)
            log(f"decode c4: graph step {dec['step_us']:.2f} us, fused {dec['fused_us']:.2f} us "
                f"({dec['fused_gbs']:.0f} GB/s; caches cycled {dec['cold_us']:.2f} us), split "
                f"{dec['split_us']:.2f} us (caches cycled {dec['split_cold_us']:.2f} us)")
        return 0

    log("prefill c3 ...")
    pre = bench_prefill(torch, ga, args.steps, args.warmup, gen)
    log(f"prefill c3: {pre['ms']:.3f} ms/launch, {pre['tflops']:.1f} TFLOP/s (static grid {pre['static_ms']:.3f} ms)")
    log("prefill split-K c3 ...")
    psp = bench_prefill_split(torch, ga, pre, args.steps)
    log(f"prefill split-K c3: split {psp['ms'] * 1e3:.1f} us + merge {psp['merge_ms'] * 1e3:.1f} us, "
        f"{psp['tflops']:.1f} TFLOP/s, max |split - unsplit| {psp['max_diff_vs_unsplit']:.2e}")
    log("mfma probe ...")
    mp = bench_mfma_probe(torch)
    log(f"mfma probe: QK operands {mp['qk']:.0f}, PV operands {mp['pv']:.0f}, "
        f"mix {mp['mix']:.0f} TFLOP/s; prefill = {pre['tflops'] / mp['mix']:.3f} of the mix")
    hp = bench_hbm_probe(torch)
    log(f"hbm read probe: {hp['gbs']:.0f} GB/s over {hp['bytes'] >> 30} GiB")
    cp = bench_hbm_copy_probe(torch)
    log(f"hbm copy probe: {cp['gbs']:.0f} GB/s read + write")
    log("c1 ...")
    c1 = bench_prefill_c1(torch, ga, gen)
    log(f"c1: attention {c1['attn_us']:.2f} us ({c1['tflops']:.1f} TFLOP/s), norm "
        f"{c1['norm_us']:.2f} us ({c1['norm_gbs']:.0f} GB/s)")
    log("qk_norm_rope c3 ...")
    nrm = bench_norm(torch, ga, args.steps, args.warmup, gen)
    log(f"norm c3: {nrm['ms'] * 1e3:.1f} us, {nrm['gbs']:.0f} GB/s; cycled "
                f"{nrm['cold_ms'] * 1e3:.1f} us, {nrm['cold_gbs']:.0f} GB/s")
    kvu = bench_kv_update(torch, ga, args.steps, args.warmup, gen)
    log(f"kv update c3: {kvu['ms'] * 1e3:.1f} us, {kvu['gbs']:.0f} GB/s; cycled "
                f"{kvu['cold_ms'] * 1e3:.1f} us, {kvu['cold_gbs']:.0f} GB/s")
    log("c5 ...")
    c5 = bench_c5(torch, ga, gen)
    log(f"c5: prefill {c5['ms']:.2f} ms ({c5['tflops']:.1f} TFLOP/s); split-K "
        f"{c5['split_ms']:.2f} + {c5['merge_ms']:.2f} ms ({c5['split_tflops']:.1f} TFLOP/s); "
        f"{c5['decode_steps']} decode steps {c5['decode_us']:.2f} us/step "
        f"({c5['decode_gbs']:.0f} GB/s)")
    log("decode c4 ...")
    dec = bench_decode(torch, ga, 64, 8, 32768, args.decode_replays, 20, gen, 200)
    dec_layers = bench_decode_layers_graph(torch, ga, gen, 64, 8, 32768, 4, 100)
    log(f"decode c4: graph step {dec['step_us']:.2f} us ({dec['step_gbs']:.0f} GB/s); 4-layer "
        f"graph {dec_layers['us']:.2f} us/layer ({dec_layers['gbs']:.0f} GB/s); fused kernel "
        f"{dec['fused_us']:.2f} us (caches cycled {dec['cold_us']:.2f} us, "
        f"{dec['cold_gbs']:.0f} GB/s); split {dec['split_us']:.2f} us (caches cycled "
        f"{dec['split_cold_us']:.2f} us); merge {dec['merge_us']:.2f} us, NKS={dec['num_splits']}")
    graph_default = measure_graph_step_default_runtime(args.decode_replays, log)
    log("decode Qwen3-4B 32K ...")
    dec4b = bench_decode(torch, ga, 32, 8, 32768, 200, 20, gen, 200)
    dec4b_layers = bench_decode_layers_graph(torch, ga, gen, 32, 8, 32768, 4, 100)
    log(f"decode 4B ctx 32768: fused kernel caches cycled {dec4b['cold_us']:.2f} us "
        f"({dec4b['cold_gbs']:.0f} GB/s), 4-layer graph {dec4b_layers['us']:.2f} us/layer")
    log("decode c2 ...")
    dec2 = bench_decode(torch, ga, 32, 8, 4096, 200, 20, gen, 200, cold_caches=24)
    dec2_layers = bench_decode_layers_graph(torch, ga, gen, 32, 8, 4096, 24, 40)
    log(f"decode c2: graph step {dec2['step_us']:.2f} us, fused {dec2['fused_us']:.2f} us "
        f"(caches cycled {dec2['cold_us']:.2f} us), split {dec2['split_us']:.2f} us, 24-layer "
        f"graph {dec2_layers['us']:.2f} us/layer")
    log("decode layer ops c4 ...")
    dl = bench_decode_layer(torch, ga, args.steps, gen)
    log("decode layer c4: " + ", ".join(
        f"{k} {v['us']:.2f} us" + (f" ({v['gbs']:.0f} GB/s)" if "gbs" in v else "")
        for k, v in dl.items()))
    log("token step c4 ...")
    ts = bench_token_step(torch, ga, gen)
    log(f"token step c4 ({ts['layers']} layers, ctx {ts['ctx']}): {ts['ms']:.3f} ms/token, "
        f"{ts['tokens_per_s']:.1f} tok/s, {ts['gbs']:.0f} GB/s")
    t4 = bench_token_step(torch, ga, gen, model=QWEN3_4B)
    log(f"token step Qwen3-4B ({t4['layers']} layers, ctx {t4['ctx']}): {t4['ms']:.3f} ms/token, "
        f"{t4['tokens_per_s']:.1f} tok/s, {t4['gbs']:.0f} GB/s")

    log("prefill c3 in the settled power state ...")
    steady = bench_prefill_steady(torch, ga, pre, args.steps)
    log(f"prefill c3 after {steady['sustain']} untimed launches: {steady['ms']:.3f} ms/launch, "
        f"{steady['tflops']:.1f} TFLOP/s (headline window: {pre['ms']:.3f} ms)")
    log("power and clocks: c3 prefill, then the MFMA probe ...")
    pw = bench_power_state(torch, ga, pre)
    if pw is None:
        log("power and clocks: amd-smi unavailable")
    else:
        for k in ("prefill_c3", "mfma_probe"):
            if k in pw:
                e = pw[k]
                log(f"{k}: {e['socket_power_w']:.0f} W, gfx clocks {min(e['gfx_clock_mhz']):.0f}-"
                    f"{max(e['gfx_clock_mhz']):.0f} MHz, {e['frac_of_peak_at_clock']:.3f} of the "
                    f"fp16 peak at that clock ({e['fp16_dense_peak_at_clock']:.0f} TFLOP/s)")

    cpu = None
    if not args.no_cpu_baseline:
        threads, visible = host_threads()
        log(f"cpu baseline ({threads} threads of {visible} visible, and 1 thread) ...")
        cpu = cpu_baselines(torch, pre, dec, c5, c1)
        log(f"cpu: c3 {cpu['c3']['value'] * 1e3:.2f} GFLOP/s ({cpu['c3']['single_thread_value'] * 1e3:.2f} "
            f"on 1 thread), c4 {cpu['c4']['value']:.2f} GB/s, c5 {cpu['c5']['value'] * 1e3:.2f} "
            f"GFLOP/s (extrapolated), c5 decode {cpu['c5_decode']['value']:.2f} GB/s")

    def rl(bound, achieved, peak, unit, traffic=None):
        return {"bound": bound, "achieved": round(achieved, 2), "peak": peak, "unit": unit,
                "frac": round(achieved / peak, 4), "traffic": traffic}

    def cpu_entry(key):
        if cpu is None:
            return None
        e = dict(cpu[key])
        e.setdefault("kind", "port")
        e["host_cpus_visible"] = cpu["host_cpus_visible"]
        return {k: (round(v, 6) if isinstance(v, float) else v) for k, v in e.items()}

    line = {
        "metric": METRIC,
        "value": round(pre["tflops"], 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(pre["ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic",
        "config": {"workload": "c3: Qwen3-4B causal prefill attention, batch 1, S=8192, "
                               "32 Q / 8 KV heads, head_dim 128, f16 (fp32 accumulation)",
                   "seq_len": pre["S"], "num_q_heads": pre["hq"], "num_kv_heads": pre["hkv"],
                   "head_dim": D, "flops_per_step": pre["flops"],
                   "entry_point": "grout_attn_prefill_sched (dynamic per-XCD schedule)",
                   "static_grid_ms_per_step": round(pre["static_ms"], 4),
                   "static_grid_TFLOP/s": round(pre["flops"] / (pre["static_ms"] * 1e-3) / 1e12, 2)},
        "roofline": rl("mfma", pre["tflops"], PEAK_TFLOPS_F16, "TFLOP/s",
                       traffic=round(PMC_TRAFFIC_BYTES["attn_prefill_c3"])),
        "cpu_baseline": cpu_entry("c3"),
        # What the matrix cores sustain on this GPU for operands distributed like
        # the prefill kernel's (MFMAs only, no memory or softmax work).
        "mfma_ceiling_probe": {
            "unit": "TFLOP/s", "qk_operands": round(mp["qk"], 1), "pv_operands": round(mp["pv"], 1),
            "mix": round(mp["mix"], 1), "frac_of_nominal_peak": round(mp["mix"] / PEAK_TFLOPS_F16, 4),
            "prefill_frac_of_mix": round(pre["tflops"] / mp["mix"], 4),
            "source": "bench_probes/mfma_ceiling.hip"},
        # What a plain streaming read kernel sustains on this GPU (cache-cold, 4 GiB).
        "hbm_read_probe": {"unit": "GB/s", "value": round(hp["gbs"], 1),
                           "frac_of_peak": round(hp["gbs"] / PEAK_HBM_GBS, 4),
                           "workgroups_per_cu": hp["workgroups_per_cu"],
                           "source": "bench_probes/hbm_read.hip"},
        # Bytes read + bytes written by a plain streaming copy: the ceiling of the
        # read-and-write kernels (qk_norm_rope_c3, kv_cache_update_c3).
        "hbm_copy_probe": {"unit": "GB/s", "value": round(cp["gbs"], 1),
                           "frac_of_peak": round(cp["gbs"] / PEAK_HBM_GBS, 4),
                           "workgroups_per_cu": cp["workgroups_per_cu"],
                           "source": "bench_probes/hbm_copy.hip"},
        "decode": {
            "workload": "c4: Qwen3-32B decode step, 64 Q / 8 KV heads, context 32768, "
                        f"hipGraph x{dec['replays']} of the fused step (norm/RoPE/KV write + "
                        "split + merge, one kernel)",
            "value": round(dec["step_gbs"], 1), "unit": "GB/s",
            "us_per_step": round(dec["step_us"], 3), "num_splits": dec["num_splits"],
            # The roofline is the fused kernel with four layers' caches cycled
            # (none served from the 256 MB last-level cache), as in a token step.
            "roofline": rl("hbm", dec["cold_gbs"], PEAK_HBM_GBS, "GB/s",
                           traffic=round(PMC_TRAFFIC_BYTES["attn_decode_fused_c4"])),
            "fused_kernel_cold_cache_us": round(dec["cold_us"], 3),
            "fused_kernel_warm_us": round(dec["fused_us"], 3),
            "graph_step_cold_cache_us": round(dec_layers["us"], 3),
            "graph_step_cold_cache_gbs": round(dec_layers["gbs"], 1),
            "graph_step_cold_cache_frac_of_hbm_peak": round(dec_layers["gbs"] / PEAK_HBM_GBS, 4),
            "graph_step_cold_cache_note": "4 layers' fused steps (4 caches, 552 MB) in one "
                                          "hipGraph, replay time / 4",
            "graph_step_default_runtime_us": graph_default,
            "hip_graph_packet_capture": packet_capture,
            "standalone_split_us": round(dec["split_us"], 3),
            "standalone_split_cold_cache_us": round(dec["split_cold_us"], 3),
            "standalone_split_cold_cache_frac_of_hbm_peak": round(
                dec["bytes_step"] / (dec["split_cold_us"] * 1e-6) / 1e9 / PEAK_HBM_GBS, 4),
            "standalone_merge_us": round(dec["merge_us"], 3),
            "step_frac_of_hbm_peak": round(dec["step_gbs"] / PEAK_HBM_GBS, 4),
            "fused_kernel_cold_cache_frac_of_read_probe": round(dec["cold_gbs"] / hp["gbs"], 4),
            "cpu_baseline": cpu_entry("c4"),
        },
        "decode_qwen3_4b_32k": {
            "workload": "Qwen3-4B decode step (32 Q / 8 KV heads), context 32768: the north "
                        "star's decode target shape",
            "fused_kernel_cold_cache_us": round(dec4b["cold_us"], 3),
            "roofline": rl("hbm", dec4b["cold_gbs"], PEAK_HBM_GBS, "GB/s"),
            "graph_step_cold_cache_us": round(dec4b_layers["us"], 3),
            "graph_step_cold_cache_frac_of_hbm_peak": round(dec4b_layers["gbs"] / PEAK_HBM_GBS, 4),
            "graph_step_warm_us": round(dec4b["step_us"], 3),
            "num_splits": dec4b["num_splits"]},
        "c5": {
            "workload": "Qwen3-32B causal prefill, S=32768, 64 Q / 8 KV heads, 1% of K rows x8, "
                        f"then {c5['decode_steps']} graph-replayed decode steps on the same cache",
            "prefill_ms": round(c5["ms"], 3),
            "prefill_static_grid_ms": round(c5["static_ms"], 3),
            "roofline": rl("mfma", c5["tflops"], PEAK_TFLOPS_F16, "TFLOP/s"),
            "prefill_flops": c5["flops"], "outlier_k_rows": c5["n_outlier_rows"],
            "split_k": {"num_splits": c5["split"][0], "block_m": c5["split"][1],
                        "block_n": c5["split"][2], "split_ms": round(c5["split_ms"], 3),
                        "merge_ms": round(c5["merge_ms"], 3),
                        "TFLOP/s": round(c5["split_tflops"], 1),
                        "vs_unsplit": round(c5["ms"] / (c5["split_ms"] + c5["merge_ms"]), 4),
                        "max_abs_diff_vs_unsplit": c5["split_max_diff"]},
            "decode_us_per_step": round(c5["decode_us"], 3),
            "decode_roofline": rl("hbm", c5["decode_gbs"], PEAK_HBM_GBS, "GB/s"),
            "decode_num_splits": c5["decode_splits"],
            "cpu_baseline": cpu_entry("c5"),
            "cpu_baseline_decode": cpu_entry("c5_decode"),
        },
        "c1": {
            "workload": "Qwen3-0.6B layer, S=512, 16 Q / 8 KV heads: fused QK norm/RoPE/KV "
                        "write then causal prefill attention (launch-bound sizes)",
            "attn_us": round(c1["attn_us"], 3),
            "roofline": rl("mfma", c1["tflops"], PEAK_TFLOPS_F16, "TFLOP/s"),
            "norm_us": round(c1["norm_us"], 3),
            "norm_roofline": rl("hbm", c1["norm_gbs"], PEAK_HBM_GBS, "GB/s"),
            "cpu_baseline": cpu_entry("c1"),
        },
        "decode_c2": {
            "workload": "c2: Qwen3-4B decode step, 32 Q / 8 KV heads, context 4096",
            "us_per_step": round(dec2["step_us"], 3),
            "fused_kernel_warm_us": round(dec2["fused_us"], 3),
            "fused_kernel_cold_cache_us": round(dec2["cold_us"], 3),
            "roofline": rl("hbm", dec2["cold_gbs"], PEAK_HBM_GBS, "GB/s"),
            "graph_step_cold_cache_us": round(dec2_layers["us"], 3),
            "graph_step_cold_cache_note": "24 layers' fused steps in one hipGraph, replay "
                                          "time / 24",
            "standalone_split_us": round(dec2["split_us"], 3),
            "num_splits": dec2["num_splits"]},
        "prefill_split_c3": {
            "split_us": round(psp["ms"] * 1e3, 2), "merge_us": round(psp["merge_ms"] * 1e3, 2),
            "TFLOP/s": round(psp["tflops"], 1), "num_splits": psp["num_splits"],
            "block_m": psp["block_m"], "block_n": psp["block_n"], "group": psp["group"],
            "max_abs_diff_vs_unsplit": psp["max_diff_vs_unsplit"]},
        "decode_layer_c4": {
            **{nm: {"m": dl[nm]["m"], "k": dl[nm]["k"], "us": round(dl[nm]["us"], 2),
                    "GB/s": round(dl[nm]["gbs"], 1),
                    "frac_of_hbm_peak": round(dl[nm]["gbs"] / PEAK_HBM_GBS, 4)}
               for nm in ("qkv_proj", "o_proj", "lm_head")},
            "add_rms_norm_us": round(dl["add_rms_norm"]["us"], 2),
            "argmax_us": round(dl["argmax"]["us"], 2)},
        "token_step_c4": {
            "workload": f"Qwen3-32B-shaped decode token step, {ts['layers']} layers, every KV "
                        f"cache at context {ts['ctx']}, one hipGraph per token (embedding .. "
                        "argmax), random f16 weights",
            "ms_per_token": round(ts["ms"], 3), "tokens_per_s": round(ts["tokens_per_s"], 2),
            "bytes_per_token": ts["bytes"], "GB/s": round(ts["gbs"], 1),
            "frac_of_hbm_peak": round(ts["gbs"] / PEAK_HBM_GBS, 4),
            "num_splits": ts["num_splits"], "steps": ts["steps"]},
        "token_step_qwen3_4b": {
            "workload": f"Qwen3-4B-shaped decode token step (the north star's model: hidden "
                        f"2560, 32 Q / 8 KV heads, intermediate 9728), {t4['layers']} layers, "
                        f"every KV cache at context {t4['ctx']}, one hipGraph per token, random "
                        "f16 weights",
            "ms_per_token": round(t4["ms"], 3), "tokens_per_s": round(t4["tokens_per_s"], 2),
            "bytes_per_token": t4["bytes"], "GB/s": round(t4["gbs"], 1),
            "frac_of_hbm_peak": round(t4["gbs"] / PEAK_HBM_GBS, 4),
            "num_splits": t4["num_splits"], "steps": t4["steps"]},
        "prefill_c3_steady_state": {
            "note": "the same c3 launches after the bench's other legs and "
                    f"{steady['sustain']} more untimed launches, once the GPU's power "
                    "management has settled; the headline value keeps the contract's "
                    "warmup count",
            "ms_per_step": round(steady["ms"], 4), "TFLOP/s": round(steady["tflops"], 2),
            "frac_of_fp16_peak": round(steady["tflops"] / PEAK_TFLOPS_F16, 4),
            "untimed_launches_before": steady["sustain"], "steps": args.steps},
        # Board power and shader clocks while c3 and the MFMA probe run for a few
        # seconds each: both sit at the board's power limit, below the 2.4 GHz
        # the nominal peak assumes.
        "power_state": pw,
        # us/GB/s: one set of buffers back to back (the last-level cache serves part
        # of it); cold_*: buffer sets cycled past that cache, all traffic from HBM.
        "qk_norm_rope_c3": {"us": round(nrm["ms"] * 1e3, 2), "GB/s": round(nrm["gbs"], 1),
                            "frac_of_hbm_peak": round(nrm["gbs"] / PEAK_HBM_GBS, 4),
                            "cold_us": round(nrm["cold_ms"] * 1e3, 2),
                            "cold_GB/s": round(nrm["cold_gbs"], 1),
                            "cold_frac_of_hbm_peak": round(nrm["cold_gbs"] / PEAK_HBM_GBS, 4)},
        "kv_cache_update_c3": {"us": round(kvu["ms"] * 1e3, 2), "GB/s": round(kvu["gbs"], 1),
                               "frac_of_hbm_peak": round(kvu["gbs"] / PEAK_HBM_GBS, 4),
                               "cold_us": round(kvu["cold_ms"] * 1e3, 2),
                               "cold_GB/s": round(kvu["cold_gbs"], 1),
                               "cold_frac_of_hbm_peak": round(kvu["cold_gbs"] / PEAK_HBM_GBS, 4)},
    }
    print(json.dumps(line), flush=True)
    return 0


def measure_graph_step_default_runtime(replays: int, log):
    """The c4 graph step (1000 replays of the one-kernel graph) under the HIP
    runtime's default graph packet capture: the setting is read when HIP
    initialises, so this runs bench.py once more as a child process with the
    variable removed from its environment.  Returns microseconds per step, or
    None when the child fails (its output is logged)."""
    import subprocess

    env = dict(os.environ)
    env.pop(GRAPH_PACKET_ENV, None)
    cmd = [sys.executable, os.path.abspath(__file__), "--only", "decode-graph-step",
           "--hip-default-graph-capture", "--decode-replays", str(replays)]
    r = subprocess.run(cmd, env=env, capture_output=True, text=True, timeout=300)
    for ln in r.stdout.splitlines()[::-1]:
        if ln.startswith("{"):
            v = json.loads(ln)["graph_step_us"]
            log(f"c4 graph step with the HIP runtime's default graph capture: {v:.2f} us")
            return v
    log(f"default-runtime graph step failed (rc {r.returncode}): {r.stderr[-400:]}")
    return None


if __name__ == "__main__":
    sys.exit(main())
