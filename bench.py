#!/usr/bin/env python3
"""Benchmark of the Qwen3 attention hot path on one MI355X.

Headline (BASELINE.json metric): prefill attention TFLOP/s as a fraction of the
fp16 dense MFMA peak, and decode attention GB/s as a fraction of HBM peak.

  value   = config c3: Qwen3-4B causal prefill attention, batch 1, S=8192,
            32 Q / 8 KV heads, head_dim 128, f16 in / f32 accumulate.
            One step = one grout_attn_prefill launch; inputs already in HBM.
  decode  = config c4: Qwen3-32B decode step, 64 Q / 8 KV heads, context
            32768, {fused norm/RoPE/KV write, split-K decode, merge} captured
            in a hipGraph and replayed 1000x with only the position updated.
  also    = c3's fused QK norm/RoPE/KV write (HBM-bound) and c2 (Qwen3-4B
            decode at context 4096).

Kernel durations come from HIP events recorded on the launch stream: around
each launch for prefill, and around a run of back-to-back launches (divided by
the count) for the microsecond-scale decode and norm kernels, whose per-launch
event pairs would add the launch latency.  The CPU baseline is the oracle (a C port of the reference's fp32
CPU attention, benchmarks/src/bin/attention_microbench.rs:665-702) run on a
bounded row sample of the same inputs.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

# HIP runtime setting for the decode-graph replays, read when HIP initialises
# (so before torch is imported): with the runtime's graph packet capture on, each
# replay of the one-kernel decode graph costs ~4 us more GPU time than the same
# kernel launched directly (measured 34.0 vs 30.2 us per step); with it off a
# replay costs what a launch costs.  An explicit setting in the environment wins.
GRAPH_PACKET_CAPTURE = os.environ.setdefault("DEBUG_CLR_GRAPH_PACKET_CAPTURE", "0")

METRIC = ("prefill attn TFLOP/s (% fp16 MFMA peak); decode attn GB/s (% HBM peak), 1 GPU")
PEAK_TFLOPS_F16 = 2516.6   # 256 CU x 4096 FLOP/clk x 2.4 GHz (dense fp16 MFMA)
PEAK_HBM_GBS = 8000.0      # HBM3E
# HBM bytes per launch from rocprofv3 --pmc FETCH_SIZE (x2.0) and WRITE_SIZE (x1.0), the
# scales read off a 1 GiB copy; the runs and figures are in profiles/*.txt.
PMC_TRAFFIC_BYTES = {
    "attn_prefill_c3": (71767.0 * 2.0 + 65536.0) * 1024,
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


def bench_prefill(torch, ga, steps, warmup, gen):
    hq, hkv, S = 32, 8, 8192
    q = torch.randn((S, hq, D), device="cuda", generator=gen, dtype=torch.float32).half()
    kc = torch.randn((hkv, S, D), device="cuda", generator=gen, dtype=torch.float32).half()
    vc = torch.randn((hkv, S, D), device="cuda", generator=gen, dtype=torch.float32).half()
    out = torch.empty_like(q)
    fn = lambda: ga.attend_prefill(q, kc, vc, out, 0)  # noqa: E731
    ms, wall = time_region(torch, fn, steps, warmup)
    assert torch.isfinite(out).all().item(), "non-finite prefill output"
    flops = prefill_flops(hq, S)
    tflops = flops / (ms * 1e-3) / 1e12
    return dict(q=q, kc=kc, vc=vc, out=out, ms=ms, wall_ms=wall, tflops=tflops, flops=flops,
                hq=hq, hkv=hkv, S=S)


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
    hq, hkv, S = 32, 8, 8192
    q = torch.randn((S, hq, D), device="cuda", generator=gen).half()
    k = torch.randn((S, hkv, D), device="cuda", generator=gen).half()
    v = torch.randn((S, hkv, D), device="cuda", generator=gen).half()
    qw = (1 + 0.1 * torch.randn((D,), device="cuda", generator=gen)).half()
    kw = (1 + 0.1 * torch.randn((D,), device="cuda", generator=gen)).half()
    inv = ga.build_inv_freq(THETA).cuda()
    kc = torch.zeros((hkv, S, D), device="cuda", dtype=torch.float16)
    vc = torch.zeros_like(kc)
    out = torch.empty_like(q)
    fn = lambda: ga.qk_norm_rope_kv_prefill(q, k, v, qw, kw, inv, out, kc, vc, EPS, 0)  # noqa
    ms = time_back_to_back(torch, fn, max(steps, 50), warmup)
    nb = norm_bytes(hq, hkv, S)
    return dict(ms=ms, bytes=nb, gbs=nb / (ms * 1e-3) / 1e9)


def bench_kv_update(torch, ga, steps, warmup, gen):
    """kv_cache_update_seq at c3 shapes: 8192 rows x 8 KV heads of K and V into
    a [8, 8192, 128] cache (read 33.6 MB, write 33.6 MB)."""
    hkv, S = 8, 8192
    nk = torch.randn((S, hkv, D), device="cuda", generator=gen).half()
    nv = torch.randn((S, hkv, D), device="cuda", generator=gen).half()
    kc = torch.zeros((hkv, S, D), device="cuda", dtype=torch.float16)
    vc = torch.zeros_like(kc)
    ga.kv_cache_update_seq(nk, nv, kc, vc, 0)  # argument checks of the Python mirror once
    # Back to back through the C entry point: the ~12 us kernel outruns the
    # Python mirror's per-call cost.
    L = ga.lib()
    args = (nk.data_ptr(), nv.data_ptr(), kc.data_ptr(), vc.data_ptr(), 0, S, hkv, D, S,
            torch.cuda.current_stream().cuda_stream)
    fn = lambda: L.grout_kv_cache_update_seq(*args)  # noqa: E731
    ms = time_back_to_back(torch, fn, max(steps, 50), warmup)
    nb = 2 * 2 * S * hkv * D * 2
    return dict(ms=ms, bytes=nb, gbs=nb / (ms * 1e-3) / 1e9)


def bench_decode(torch, ga, hq, hkv, ctx, replays, warmup, gen, split_steps):
    """Graph replay of {norm/RoPE/KV write, split, merge} at positions ctx..ctx+replays-1,
    plus event-timed eager launches of the split kernel alone at position ctx."""
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
    scale_bits = int(torch.tensor([1.0 / math.sqrt(D)], dtype=torch.float16).view(torch.int16)
                     .item()) & 0xFFFF
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

    # The fused step alone (the graph's only kernel), eager at position ctx
    # (s_kv = ctx + 1, position not advanced), back-to-back launches; then the
    # standalone split and merge ops of the same shape.
    counters = ga.decode_counters(hkv)
    pos_t.fill_(ctx)
    with torch.cuda.stream(s):
        ffn = lambda: ga.decode_fused(qkv, qw, kw, inv, q_out, kc, vc, att, lse, attn_out,  # noqa
                                      counters, pos_t, EPS, scale_bits, hq, hkv)
        fused_us = 1e3 * time_back_to_back(torch, ffn, split_steps, 10, stream=s)
        q_grouped = q_out[:hq].view(hkv, G, D)
        fn = lambda: ga.fmha_decode_gqa_split(q_grouped, kc, vc, att, lse, scale_bits, pos_t)  # noqa
        split_us = 1e3 * time_back_to_back(torch, fn, split_steps, 10, stream=s)
        # The same fused step cycling through 4 layers' caches (552 MB), so no
        # launch finds its K/V in the 256 MB last-level cache: the situation of
        # a real token step, where 63 other layers run between two reads of one
        # layer's cache.
        kcs = [kc] + [torch.randn_like(kc) for _ in range(3)]
        vcs = [vc] + [torch.randn_like(vc) for _ in range(3)]
        it = [0]

        def cold():
            it[0] += 1
            c = it[0] % 4
            ga.decode_fused(qkv, qw, kw, inv, q_out, kcs[c], vcs[c], att, lse, attn_out,
                            counters, pos_t, EPS, scale_bits, hq, hkv)
        cold_us = 1e3 * time_back_to_back(torch, cold, split_steps, 12, stream=s)

        def split_cold():
            it[0] += 1
            c = it[0] % 4
            ga.fmha_decode_gqa_split(q_grouped, kcs[c], vcs[c], att, lse, scale_bits, pos_t)
        split_cold_us = 1e3 * time_back_to_back(torch, split_cold, split_steps, 12, stream=s)
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
    args = (r.data_ptr(), x.data_ptr(), w.data_ptr(), o.data_ptr(), ro.data_ptr(), EPS, n, st)
    res["add_rms_norm"] = dict(n=n, us=1e3 * time_back_to_back(
        torch, lambda: L.grout_add_rms_norm_decode(*args), max(steps, 200), 20))
    v = 151936
    lg = torch.randn((v,), device="cuda", generator=gen).half()
    bm, bi = ga.argmax_scratch(v)
    tok = torch.empty((1,), device="cuda", dtype=torch.int32)
    aargs = (lg.data_ptr(), bm.data_ptr(), bi.data_ptr(), tok.data_ptr(), v, st)
    res["argmax"] = dict(n=v, us=1e3 * time_back_to_back(
        torch, lambda: L.grout_argmax_f16(*aargs), max(steps, 200), 20))
    assert int(tok.item()) == int(torch.argmax(lg.float()).item()), "argmax mismatch"
    return res


def bench_token_step(torch, ga, gen, layers=64, ctx=32768, steps=20):
    """The whole Qwen3-32B decode token step (hidden 5120, 64 Q / 8 KV heads,
    intermediate 25600, vocab 151936, `layers` layers) as one hipGraph, every
    layer's KV cache holding `ctx` tokens: `steps` replays issued back to back
    from C, each embedding the token the previous one picked.  Random f16
    weights; bytes per token = every weight matrix + the KV read and written."""
    hidden, inter, vocab, hq, hkv = 5120, 25600, 151936, 64, 8
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
    over a buffer far larger than the 256 MB last-level cache: the practical ceiling of the
    HBM-bound kernels.  GB/s (1e9 bytes)."""
    import ctypes

    import bench_probes

    lib = ctypes.CDLL(bench_probes.lib_path())
    fn = lib.grout_probe_hbm_read
    fn.restype = ctypes.c_int32
    fn.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int32, ctypes.c_void_p]
    nbytes = gib << 30
    src = torch.empty((nbytes,), dtype=torch.uint8, device="cuda").fill_(1)
    blocks = 8 * torch.cuda.get_device_properties(0).multi_processor_count
    out = torch.empty((blocks * 256,), dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream()
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
    del src
    torch.cuda.empty_cache()
    return dict(gbs=gbs, bytes=nbytes, blocks=blocks)


def cpu_baseline_prefill(torch, pre, threads: int):
    """Oracle fp32 attention over every query row of the c3 inputs (about 10 s on 16 cores)."""
    import oracle

    q = pre["q"].cpu().numpy()
    kc = pre["kc"].cpu().numpy()
    vc = pre["vc"].cpu().numpy()
    S, hq = pre["S"], pre["hq"]
    step, begin = 1, 0
    t0 = time.perf_counter()
    oracle.attn_prefill_f32(q, kc, vc, 1.0 / math.sqrt(D), S, 0, row_begin=begin,
                            row_step=step, nthreads=threads)
    dt = time.perf_counter() - t0
    rows = range(begin, S, step)
    flops = sum(2.0 * 2.0 * D * hq * (m + 1) for m in rows)
    return dict(value=flops / dt / 1e12, unit="TFLOP/s", cores=threads, kind="port",
                sample=f"c3 inputs, query rows {begin}::{step} ({len(rows)} of {S}) x {hq} "
                       f"heads, {dt:.1f} s; oracle/grout_oracle.c go_attn_prefill_f32 "
                       f"(fp32, two-pass softmax), OpenMP over (row, head)")


def cpu_baseline_decode(torch, dec, threads: int):
    import oracle

    hq, hkv, ctx = dec["hq"], dec["hkv"], dec["ctx"]
    q = dec["q"].cpu().numpy().reshape(1, hq, D)
    kc = dec["kc"][:, :ctx + 1].contiguous().cpu().numpy()
    vc = dec["vc"][:, :ctx + 1].contiguous().cpu().numpy()
    t0 = time.perf_counter()
    oracle.attn_prefill_f32(q, kc, vc, 0.08837890625, ctx + 1, ctx, nthreads=threads)
    dt = time.perf_counter() - t0
    return dict(value=decode_bytes(hq, hkv, ctx + 1) / dt / 1e9, unit="GB/s", cores=threads,
                kind="port", sample=f"one c4 decode step (s_kv={ctx + 1}, {hq} heads), "
                                    f"{dt * 1e3:.0f} ms, fp32 oracle")


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
                                       "mfma-probe", "decode-layer", "token-step", "hbm-probe"],
                    default="all",
                    help="run one workload only (for profiling runs); prints no JSON line")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run a plain 1 GiB device-to-device copy (reads and writes 1 GiB) "
                         "to scale rocprofv3 FETCH_SIZE/WRITE_SIZE readings, then exit")
    args = ap.parse_args(argv)
    if args.gpus != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(attention shards by KV head with no communication; see DESIGN.md).",
              file=sys.stderr)
        return 2

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
            log(f"prefill c3: {pre['ms']:.3f} ms/launch, {pre['tflops']:.1f} TFLOP/s")
        elif args.only == "norm":
            nrm = bench_norm(torch, ga, args.steps, args.warmup, gen)
            log(f"norm c3: {nrm['ms'] * 1e3:.1f} us, {nrm['gbs']:.0f} GB/s")
        elif args.only == "kv":
            kvu = bench_kv_update(torch, ga, args.steps, args.warmup, gen)
            log(f"kv update c3: {kvu['ms'] * 1e3:.1f} us, {kvu['gbs']:.0f} GB/s")
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
        elif args.only == "hbm-probe":
            hp = bench_hbm_probe(torch)
            log(f"hbm read probe: {hp['gbs']:.0f} GB/s over {hp['bytes'] >> 30} GiB")
        elif args.only == "mfma-probe":
            mp = bench_mfma_probe(torch)
            log(f"mfma probe: QK operands {mp['qk']:.0f}, PV operands {mp['pv']:.0f}, "
                f"mix {mp['mix']:.0f} TFLOP/s")
        else:
            dec = bench_decode(torch, ga, 64, 8, 32768, args.decode_replays, args.warmup, gen,
                               args.steps)
            log(f"decode c4: graph step {dec['step_us']:.2f} us, fused {dec['fused_us']:.2f} us "
                f"({dec['fused_gbs']:.0f} GB/s; caches cycled {dec['cold_us']:.2f} us), split "
                f"{dec['split_us']:.2f} us (caches cycled {dec['split_cold_us']:.2f} us)")
        return 0

    log("prefill c3 ...")
    pre = bench_prefill(torch, ga, args.steps, args.warmup, gen)
    log(f"prefill c3: {pre['ms']:.3f} ms/launch, {pre['tflops']:.1f} TFLOP/s")
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
    log("qk_norm_rope c3 ...")
    nrm = bench_norm(torch, ga, args.steps, args.warmup, gen)
    log(f"norm c3: {nrm['ms'] * 1e3:.1f} us, {nrm['gbs']:.0f} GB/s")
    kvu = bench_kv_update(torch, ga, args.steps, args.warmup, gen)
    log(f"kv update c3: {kvu['ms'] * 1e3:.1f} us, {kvu['gbs']:.0f} GB/s")
    log("decode c4 ...")
    dec = bench_decode(torch, ga, 64, 8, 32768, args.decode_replays, 20, gen, 200)
    log(f"decode c4: graph step {dec['step_us']:.2f} us ({dec['step_gbs']:.0f} GB/s), "
        f"fused kernel {dec['fused_us']:.2f} us ({dec['fused_gbs']:.0f} GB/s; "
        f"caches cycled {dec['cold_us']:.2f} us, {dec['cold_gbs']:.0f} GB/s), "
        f"split {dec['split_us']:.2f} us ({dec['split_gbs']:.0f} GB/s; caches cycled "
        f"{dec['split_cold_us']:.2f} us), "
        f"merge {dec['merge_us']:.2f} us, NKS={dec['num_splits']}")
    log("decode layer ops c4 ...")
    dl = bench_decode_layer(torch, ga, args.steps, gen)
    log("decode layer c4: " + ", ".join(
        f"{k} {v['us']:.2f} us" + (f" ({v['gbs']:.0f} GB/s)" if "gbs" in v else "")
        for k, v in dl.items()))
    log("token step c4 ...")
    ts = bench_token_step(torch, ga, gen)
    log(f"token step c4 ({ts['layers']} layers, ctx {ts['ctx']}): {ts['ms']:.3f} ms/token, "
        f"{ts['tokens_per_s']:.1f} tok/s, {ts['gbs']:.0f} GB/s")
    log("decode c2 ...")
    dec2 = bench_decode(torch, ga, 32, 8, 4096, 200, 20, gen, 200)
    log(f"decode c2: graph step {dec2['step_us']:.2f} us, fused {dec2['fused_us']:.2f} us, "
        f"split {dec2['split_us']:.2f} us")

    threads = min(16, os.cpu_count() or 1)
    cpu = None
    cpu_dec = None
    if not args.no_cpu_baseline:
        log(f"cpu baseline ({threads} threads) ...")
        cpu = cpu_baseline_prefill(torch, pre, threads)
        cpu_dec = cpu_baseline_decode(torch, dec, threads)
        log(f"cpu: {cpu['value'] * 1e3:.2f} GFLOP/s prefill, {cpu_dec['value']:.2f} GB/s decode")

    def rl(bound, achieved, peak, unit, traffic=None):
        return {"bound": bound, "achieved": round(achieved, 2), "peak": peak, "unit": unit,
                "frac": round(achieved / peak, 4), "traffic": traffic}

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
                   "head_dim": D, "flops_per_step": pre["flops"]},
        "roofline": rl("mfma", pre["tflops"], PEAK_TFLOPS_F16, "TFLOP/s",
                       traffic=round(PMC_TRAFFIC_BYTES["attn_prefill_c3"])),
        "cpu_baseline": cpu,
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
                           "source": "bench_probes/hbm_read.hip"},
        "decode": {
            "workload": "c4: Qwen3-32B decode step, 64 Q / 8 KV heads, context 32768, "
                        f"hipGraph x{dec['replays']} of the fused step (norm/RoPE/KV write + "
                        "split + merge, one kernel)",
            "value": round(dec["step_gbs"], 1), "unit": "GB/s",
            "us_per_step": round(dec["step_us"], 3), "num_splits": dec["num_splits"],
            "fused_kernel_us": round(dec["fused_us"], 3),
            "fused_kernel_cold_cache_us": round(dec["cold_us"], 3),
            "fused_kernel_cold_cache_gbs": round(dec["cold_gbs"], 1),
            "standalone_split_us": round(dec["split_us"], 3),
            "standalone_split_cold_cache_us": round(dec["split_cold_us"], 3),
            "standalone_split_cold_cache_frac_of_hbm_peak": round(
                dec["bytes_step"] / (dec["split_cold_us"] * 1e-6) / 1e9 / PEAK_HBM_GBS, 4),
            "standalone_merge_us": round(dec["merge_us"], 3),
            "roofline": rl("hbm", dec["fused_gbs"], PEAK_HBM_GBS, "GB/s",
                           traffic=round(PMC_TRAFFIC_BYTES["attn_decode_fused_c4"])),
            "step_frac_of_hbm_peak": round(dec["step_gbs"] / PEAK_HBM_GBS, 4),
            "fused_kernel_frac_of_read_probe": round(dec["fused_gbs"] / hp["gbs"], 4),
            "hip_graph_packet_capture": GRAPH_PACKET_CAPTURE,
            "cpu_baseline": cpu_dec,
        },
        "prefill_split_c3": {
            "split_us": round(psp["ms"] * 1e3, 2), "merge_us": round(psp["merge_ms"] * 1e3, 2),
            "TFLOP/s": round(psp["tflops"], 1), "num_splits": psp["num_splits"],
            "block_m": psp["block_m"], "block_n": psp["block_n"], "group": psp["group"],
            "max_abs_diff_vs_unsplit": psp["max_diff_vs_unsplit"]},
        "decode_c2": {"us_per_step": round(dec2["step_us"], 3),
                      "fused_kernel_us": round(dec2["fused_us"], 3),
                      "fused_gbs": round(dec2["fused_gbs"], 1),
                      "num_splits": dec2["num_splits"]},
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
        "qk_norm_rope_c3": {"us": round(nrm["ms"] * 1e3, 2), "GB/s": round(nrm["gbs"], 1),
                            "frac_of_hbm_peak": round(nrm["gbs"] / PEAK_HBM_GBS, 4)},
        "kv_cache_update_c3": {"us": round(kvu["ms"] * 1e3, 2), "GB/s": round(kvu["gbs"], 1),
                               "frac_of_hbm_peak": round(kvu["gbs"] / PEAK_HBM_GBS, 4)},
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
