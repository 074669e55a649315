"""GPU parity of the whole Qwen3 decode token step (the graph of
src/model.rs:3118-3648 on this library's kernels) and of its two remaining
ops, embedding + RMSNorm (src/kernels.rs:693-711, 304-344) and SiLU * up
(src/kernels.rs:271-301), against the oracle.

Contract:
* embed + norm: residual_out bit-exact (a row copy), out within 1 f16 ulp;
* SiLU * up within 1 f16 ulp;
* token step (a 2-layer model, random weights): logits within 1e-2 + 1e-2|x|
  of the oracle's composed step fed the same token (its attention split on
  the fused decode step's balanced boundaries), the picked token equal to
  the argmax of the logits the GPU produced, the caches written at each step's
  position within 2e-2 of the oracle's (bit-exact elsewhere), and the device
  position advanced once per step.  Graph replays, eager steps and replays
  issued back to back from C agree to the same tolerance.
"""
import copy

import numpy as np
import pytest

import oracle
from tests._util import assert_close_attn, f16_ulp_diff, normal_f16, qwen3_tiny_model, rng

pytestmark = pytest.mark.gpu


def _dev(torch, a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


@pytest.mark.parametrize("n,vocab,tok", [(256, 1000, 7), (5120, 300, 299), (8, 3, 0),
                                         (1024, 50, 1000)])   # id past the table: last row
def test_embed_rms_norm_matches_oracle(gpu, n, vocab, tok):
    import torch
    import grout_amd

    g = rng(1300 + n)
    table = normal_f16(g, (vocab, n))
    w = (1.0 + 0.1 * g.standard_normal(n)).astype(np.float16)
    t = torch.tensor([tok], dtype=torch.int32, device="cuda")
    out = torch.full((n,), float("nan"), dtype=torch.float16, device="cuda")
    res = torch.full((n,), float("nan"), dtype=torch.float16, device="cuda")
    grout_amd.embed_rms_norm_decode(t, _dev(torch, table), _dev(torch, w), out, res, 1e-6)
    torch.cuda.synchronize()
    row = table[min(tok, vocab - 1)]
    eo, er = oracle.add_rms_norm(row, np.zeros_like(row), w, 1e-6)
    assert np.array_equal(res.cpu().numpy().view(np.uint16), row.view(np.uint16))
    assert np.array_equal(er, row)
    assert f16_ulp_diff(out.cpu().numpy(), eo).max() <= 1


@pytest.mark.parametrize("n", [8, 512, 25600, 51208])
def test_silu_mul_matches_oracle(gpu, n):
    import torch
    import grout_amd

    g = rng(1400 + n)
    gate, up = normal_f16(g, n, 4.0), normal_f16(g, n)
    gate[:4] = np.float16([0.0, 30.0, -30.0, -100.0])
    out = torch.full((n,), float("nan"), dtype=torch.float16, device="cuda")
    grout_amd.silu_mul(_dev(torch, gate), _dev(torch, up), out)
    torch.cuda.synchronize()
    assert f16_ulp_diff(out.cpu().numpy(), oracle.silu_mul(gate, up)).max() <= 1


@pytest.mark.parametrize("n,k,seed", [
    (25600, 5120, 1),   # Qwen3-32B intermediate / hidden: 8 weight rows per workgroup
    (9728, 2560, 2),    # Qwen3-4B intermediate / hidden
    (3000, 1032, 3),    # 6000 weight rows: 4 per workgroup; k not a whole unrolled chunk row
    (1001, 24, 4),      # 2002 rows: 2 per workgroup, the last one half full
    (1, 8, 5),          # one output, one chunk
])
def test_gemv_silu_mul_equals_two_launches(gpu, n, k, seed):
    """grout_gemv_silu_mul_f16 (the gate_up GEMV with SiLU * up in its epilogue, the
    token step's form) equals grout_gemv_f16 followed by grout_silu_mul_f16, bit for
    bit; both of those are held to the oracle by their own tests."""
    import torch
    import grout_amd

    g = rng(1450 + seed)
    w = normal_f16(g, (2 * n, k), 1.0 / np.sqrt(k))
    w[:4] *= np.float16(40.0)  # large gate values: silu saturates (g -> g, -> -0)
    x = normal_f16(g, k)
    dw, dx = _dev(torch, w), _dev(torch, x)
    gu = torch.empty((2 * n,), dtype=torch.float16, device="cuda")
    grout_amd.gemv_f16(dw, dx, gu)
    n8 = -(-n // 8) * 8  # silu_mul takes whole 16-byte chunks: pad with zeros
    gate = torch.zeros((n8,), dtype=torch.float16, device="cuda")
    up = torch.zeros_like(gate)
    gate[:n], up[:n] = gu[:n], gu[n:]
    ref = torch.empty_like(gate)
    grout_amd.silu_mul(gate, up, ref)
    out = torch.full((n,), float("nan"), dtype=torch.float16, device="cuda")
    grout_amd.gemv_silu_mul(dw, dx, out)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), ref[:n].view(torch.int16))


def _device_model(torch, m):
    layers = [{k: _dev(torch, v) for k, v in L.items()} for L in m["layers"]]
    return dict(layers=layers, embed_tokens=_dev(torch, m["embed_tokens"]),
                final_norm=_dev(torch, m["final_norm"]), lm_head=_dev(torch, m["lm_head"]),
                inv_freq=_dev(torch, m["inv_freq"]))


def _check_caches(dm, m, positions):
    for li, (L, R) in enumerate(zip(dm["layers"], m["layers"])):
        for key in ("k_cache", "v_cache"):
            got = L[key].cpu().numpy()
            exp = R[key]
            other = np.ones(got.shape[1], bool)
            other[list(positions)] = False
            assert np.array_equal(got[:, other], exp[:, other]), f"layer {li} {key} off-slot write"
            d = np.abs(got[:, list(positions)].astype(np.float32) - exp[:, list(positions)])
            assert d.max() < 2e-2, f"layer {li} {key} at {positions}: {d.max()}"


def test_token_step_graph_matches_oracle(gpu):
    """Graph replays, launch_step and an eager step against the oracle's composed
    step.  The fused attention balances its splits in 16-token sub-chunks, so the
    oracle composes with those boundaries; the logits of the prime step and the
    replays are also held, to the same tolerance, to the oracle on the
    reference's split boundaries."""
    import torch
    import grout_amd

    m = qwen3_tiny_model(1500)
    ref = copy.deepcopy(m)  # the oracle's own caches
    ref_r = copy.deepcopy(m)  # the oracle on the reference's split boundaries
    dm = _device_model(torch, m)
    vocab = m["embed_tokens"].shape[0]
    p0, t0, bn, ns = 20, 123, 32, 3
    token = torch.tensor([t0], dtype=torch.int32, device="cuda")
    position = torch.zeros((1,), dtype=torch.int32, device="cuda")
    logits = torch.zeros((vocab,), dtype=torch.float16, device="cuda")
    print(f"[qwen3 step] 2 layers, prime at {p0}", flush=True)
    runner = grout_amd.Qwen3DecodeRunner(
        **dm, token=token, position=position, logits=logits, num_q_heads=m["num_q_heads"],
        num_kv_heads=m["num_kv_heads"], eps=m["eps"], qk_scale_f16_bits=m["qk_scale_f16_bits"],
        num_splits=ns, block_n=bn, prime_position=p0)
    try:
        torch.cuda.synchronize()
        written = [p0]
        rl, _ = oracle.qwen3_decode_step(ref, t0, p0, bn, ns, fused_ranges=True)
        rr, _ = oracle.qwen3_decode_step(ref_r, t0, p0, bn, ns)
        gl = logits.cpu().numpy()
        assert_close_attn(gl, rl, "prime step logits", atol=1e-2, rtol=1e-2)
        assert_close_attn(gl, rr, "prime step logits (reference splits)", atol=1e-2, rtol=1e-2)
        tok = int(token.item())
        assert tok == oracle.argmax_f16(gl)
        assert int(position.item()) == p0 + 1
        # launch_step: one replay per call, the token read back.
        for i in range(1, 4):
            nxt = runner.step(p0 + i)
            rl, _ = oracle.qwen3_decode_step(ref, tok, p0 + i, bn, ns, fused_ranges=True)
            rr, _ = oracle.qwen3_decode_step(ref_r, tok, p0 + i, bn, ns)
            gl = logits.cpu().numpy()
            assert_close_attn(gl, rl, f"replay {i} logits", atol=1e-2, rtol=1e-2)
            assert_close_attn(gl, rr, f"replay {i} logits (reference splits)", atol=1e-2, rtol=1e-2)
            assert nxt == oracle.argmax_f16(gl) == int(token.item())
            tok = nxt
            written.append(p0 + i)
        assert int(position.item()) == p0 + 4
        _check_caches(dm, ref, written)
        # An eager step on the runner's stream matches the oracle the same way.
        runner.eager_step()
        torch.cuda.synchronize()
        rl, _ = oracle.qwen3_decode_step(ref, tok, p0 + 4, bn, ns, fused_ranges=True)
        gl = logits.cpu().numpy()
        assert_close_attn(gl, rl, "eager step logits", atol=1e-2, rtol=1e-2)
        tok = int(token.item())
        assert tok == oracle.argmax_f16(gl)
        # Seeding a token, then replays issued back to back from C: the oracle
        # follows the token chain the GPU picked (read from the final state).
        runner.seed_token(5)
        runner.step(p0 + 5)
        rl, _ = oracle.qwen3_decode_step(ref, 5, p0 + 5, bn, ns, fused_ranges=True)
        assert_close_attn(logits.cpu().numpy(), rl, "seeded step logits", atol=1e-2, rtol=1e-2)
        tok = int(token.item())
        runner.run(p0 + 6, 3)
        torch.cuda.synchronize()
        assert int(position.item()) == p0 + 9
        for i in range(6, 9):
            rl, t = oracle.qwen3_decode_step(ref, tok, p0 + i, bn, ns, fused_ranges=True)
            tok = t
        gl = logits.cpu().numpy()
        assert_close_attn(gl, rl, "back-to-back replay logits", atol=1e-2, rtol=1e-2)
        assert int(token.item()) == oracle.argmax_f16(gl)
        _check_caches(dm, ref, range(p0, p0 + 9))
    finally:
        runner.close()


def test_token_step_single_layer_gqa8(gpu):
    """One layer at Qwen3-32B head counts (64 Q / 8 KV heads), hidden 512."""
    import torch
    import grout_amd

    m = qwen3_tiny_model(1600, layers=1, hidden=512, hq=64, hkv=8, inter=256, vocab=4096,
                         max_seq=128, filled=100)
    ref = copy.deepcopy(m)
    dm = _device_model(torch, m)
    token = torch.tensor([77], dtype=torch.int32, device="cuda")
    position = torch.zeros((1,), dtype=torch.int32, device="cuda")
    logits = torch.zeros((4096,), dtype=torch.float16, device="cuda")
    runner = grout_amd.Qwen3DecodeRunner(
        **dm, token=token, position=position, logits=logits, num_q_heads=64, num_kv_heads=8,
        eps=m["eps"], qk_scale_f16_bits=m["qk_scale_f16_bits"], num_splits=4, block_n=32,
        prime_position=100)
    try:
        torch.cuda.synchronize()
        rl, _ = oracle.qwen3_decode_step(ref, 77, 100, 32, 4, fused_ranges=True)
        assert_close_attn(logits.cpu().numpy(), rl, "prime logits", atol=1e-2, rtol=1e-2)
        tok = int(token.item())
        nxt = runner.step(101)
        rl, _ = oracle.qwen3_decode_step(ref, tok, 101, 32, 4, fused_ranges=True)
        gl = logits.cpu().numpy()
        assert_close_attn(gl, rl, "replay logits", atol=1e-2, rtol=1e-2)
        assert nxt == oracle.argmax_f16(gl)
        _check_caches(dm, ref, [100, 101])
    finally:
        runner.close()


def test_token_step_qwen3_06b_shapes(gpu):
    """Two layers at Qwen3-0.6B shapes (config c1's model: hidden 1024, 16 Q / 8 KV heads,
    intermediate 3072) with the full 151936-token vocabulary: lm_head GEMV and argmax at
    their real sizes inside the graph."""
    import torch
    import grout_amd

    m = qwen3_tiny_model(1650, layers=2, hidden=1024, hq=16, hkv=8, inter=3072, vocab=151936,
                         max_seq=64, filled=30)
    ref = copy.deepcopy(m)
    dm = _device_model(torch, m)
    token = torch.tensor([151000], dtype=torch.int32, device="cuda")
    position = torch.zeros((1,), dtype=torch.int32, device="cuda")
    logits = torch.zeros((151936,), dtype=torch.float16, device="cuda")
    print("[qwen3 step] Qwen3-0.6B shapes, vocab 151936", flush=True)
    runner = grout_amd.Qwen3DecodeRunner(
        **dm, token=token, position=position, logits=logits, num_q_heads=16, num_kv_heads=8,
        eps=m["eps"], qk_scale_f16_bits=m["qk_scale_f16_bits"], num_splits=2, block_n=32,
        prime_position=30)
    try:
        torch.cuda.synchronize()
        tok = 151000
        for pos in (30, 31, 32):
            if pos > 30:
                runner.step(pos)
            rl, _ = oracle.qwen3_decode_step(ref, tok, pos, 32, 2, fused_ranges=True)
            gl = logits.cpu().numpy()
            assert_close_attn(gl, rl, f"position {pos} logits", atol=1e-2, rtol=1e-2)
            tok = int(token.item())
            assert tok == oracle.argmax_f16(gl)
        _check_caches(dm, ref, [30, 31, 32])
    finally:
        runner.close()


def test_runner_step_after_eager_step_writes_position(gpu):
    """step(p), an eager step (which moves the device position to p+2), then
    step(p+1): the replay runs at p+1, as launch_step writes the position on
    every step (src/model.rs:363-403).  Slot p+2 keeps its old contents."""
    import torch
    import grout_amd

    m = qwen3_tiny_model(1700, layers=1, hidden=256, hq=8, hkv=2, inter=256, vocab=512,
                         max_seq=64, filled=40)
    ref = copy.deepcopy(m)
    dm = _device_model(torch, m)
    token = torch.tensor([9], dtype=torch.int32, device="cuda")
    position = torch.zeros((1,), dtype=torch.int32, device="cuda")
    logits = torch.zeros((512,), dtype=torch.float16, device="cuda")
    runner = grout_amd.Qwen3DecodeRunner(
        **dm, token=token, position=position, logits=logits, num_q_heads=8, num_kv_heads=2,
        eps=m["eps"], qk_scale_f16_bits=m["qk_scale_f16_bits"], num_splits=3, block_n=32,
        prime_position=40)
    try:
        torch.cuda.synchronize()
        # The oracle follows the token chain the GPU picked.
        oracle.qwen3_decode_step(ref, 9, 40, 32, 3, fused_ranges=True)
        t_in = int(token.item())
        runner.step(41)
        oracle.qwen3_decode_step(ref, t_in, 41, 32, 3, fused_ranges=True)
        # Eager step at 41 + 1 = 42; the device position ends at 43.
        t_in = int(token.item())
        runner.eager_step()
        runner.stream.synchronize()
        assert int(position.item()) == 43
        oracle.qwen3_decode_step(ref, t_in, 42, 32, 3, fused_ranges=True)
        # A step at 42 again: the runner must write the position.
        t_in = int(token.item())
        nxt = runner.step(42)
        rl, _ = oracle.qwen3_decode_step(ref, t_in, 42, 32, 3, fused_ranges=True)
        gl = logits.cpu().numpy()
        assert_close_attn(gl, rl, "step after eager step", atol=1e-2, rtol=1e-2)
        assert nxt == oracle.argmax_f16(gl)
        assert int(position.item()) == 43
        _check_caches(dm, ref, [40, 41, 42])
    finally:
        runner.close()


def test_runner_picked_splits_two_kv_heads_multi_batch_merge(gpu):
    """A runner at Hkv=4, G=16 with grout_attn_decode_pick_splits' count (64 on
    256 CUs): the fused merge folds its 64 splits in two batches of partial
    rows (32 splits of 16 rows each), carrying the online max/sum across them."""
    import torch
    import grout_amd

    m = qwen3_tiny_model(1750, layers=1, hidden=256, hq=64, hkv=4, inter=256, vocab=512,
                         max_seq=4200, filled=4100)
    ref = copy.deepcopy(m)
    dm = _device_model(torch, m)
    ns = grout_amd.pick_num_splits(4200, 4)
    print(f"[qwen3 step] Hkv=4 G=16 picked splits {ns}", flush=True)
    token = torch.tensor([3], dtype=torch.int32, device="cuda")
    position = torch.zeros((1,), dtype=torch.int32, device="cuda")
    logits = torch.zeros((512,), dtype=torch.float16, device="cuda")
    runner = grout_amd.Qwen3DecodeRunner(
        **dm, token=token, position=position, logits=logits, num_q_heads=64, num_kv_heads=4,
        eps=m["eps"], qk_scale_f16_bits=m["qk_scale_f16_bits"], num_splits=ns, block_n=32,
        prime_position=4100)
    try:
        torch.cuda.synchronize()
        rl, _ = oracle.qwen3_decode_step(ref, 3, 4100, 32, ns, fused_ranges=True)
        gl = logits.cpu().numpy()
        assert_close_attn(gl, rl, "prime logits", atol=1e-2, rtol=1e-2)
        tok = int(token.item())
        assert tok == oracle.argmax_f16(gl)
        nxt = runner.step(4101)
        rl, _ = oracle.qwen3_decode_step(ref, tok, 4101, 32, ns, fused_ranges=True)
        gl = logits.cpu().numpy()
        assert_close_attn(gl, rl, "replay logits", atol=1e-2, rtol=1e-2)
        assert nxt == oracle.argmax_f16(gl)
        _check_caches(dm, ref, [4100, 4101])
    finally:
        runner.close()
