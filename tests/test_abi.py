"""CPU tests of the C-ABI boundary (no GPU, no kernel launches).

* the library loads and exports every function include/grout_attn_hip.h declares;
* each argument check returns its documented status before any HIP call, as the
  reference's ensure!s do before a launch (src/model.rs:4480-4560, 5564-5637);
* host-side helpers (RoPE table, split picking, scratch sizes) behave as specified;
* the Python mirror raises the reference's ensure! messages on bad shapes.
"""
import os
import re

import numpy as np
import pytest

import oracle

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "grout_attn_hip.h")

# Fake device addresses: never dereferenced, the checks reject the call first.
A = 0x100000        # 16-byte aligned
U = 0x100002        # misaligned


@pytest.fixture(scope="module")
def L():
    import grout_amd

    return grout_amd.lib()


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(grout_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported(L):
    import grout_amd._lib as gl

    names = header_functions()
    assert len(names) >= 20
    for name in names:
        assert hasattr(L, name), f"{name} declared in the header but not exported"
        assert name in gl.SIGNATURES, f"{name} has no ctypes signature"


def test_status_strings(L):
    import grout_amd._lib as gl

    for code, name in gl.STATUS_NAMES.items():
        text = L.grout_status_string(code).decode()
        assert text and text != "unknown status", name
    assert L.grout_status_string(-999).decode() == "unknown status"


S = None  # null stream


def prefill_norm(L, **kw):
    args = dict(q=A, k=A, v=A, qw=A, kw=A, inv=A, qo=A, kc=A, vc=A, eps=1e-6, ps=0, S=4,
                hq=4, hkv=2, D=128, MS=16)
    args.update(kw)
    return L.grout_qk_norm_rope_kv_prefill(
        args["q"], args["k"], args["v"], args["qw"], args["kw"], args["inv"], args["qo"],
        args["kc"], args["vc"], args["eps"], args["ps"], args["S"], args["hq"], args["hkv"],
        args["D"], args["MS"], S)


def test_norm_prefill_checks(L):
    assert prefill_norm(L, q=0) == -1
    assert prefill_norm(L, vc=0) == -1
    assert prefill_norm(L, k=U) == -2
    assert prefill_norm(L, D=64) == -3
    assert prefill_norm(L, hq=3, hkv=2) == -4
    assert prefill_norm(L, hkv=0) == -4
    assert prefill_norm(L, ps=13, S=4, MS=16) == -5      # 17 > max_seq_len
    assert prefill_norm(L, S=-1) == -5
    assert prefill_norm(L, eps=-1.0) == -9
    assert prefill_norm(L, eps=float("nan")) == -9
    assert prefill_norm(L, S=0) == 0                      # empty: nothing launched


def test_norm_decode_checks(L):
    f = L.grout_qk_norm_rope_kv_decode
    assert f(A, A, A, A, A, A, A, 0, 1e-6, 4, 2, 128, 16, S) == -1
    assert f(A, A, A, A, A, A, A, A + 2, 1e-6, 4, 2, 128, 16, S) == -2
    assert f(A, A, A, A, A, A, A, A, 1e-6, 4, 2, 96, 16, S) == -3
    assert f(A, A, A, A, A, A, A, A, 1e-6, 4, 3, 128, 16, S) == -4
    assert f(A, A, A, A, U, A, A, A, 1e-6, 4, 2, 128, 16, S) == -2


def test_prefill_checks(L):
    f = L.grout_attn_prefill
    ok = dict(q=A, k=A, v=A, o=A, sc=0.088, hq=4, hkv=2, D=128, ql=8, kv=8, qs=0, MS=16)

    def call(**kw):
        a = dict(ok, **kw)
        return f(a["q"], a["k"], a["v"], a["o"], a["sc"], a["hq"], a["hkv"], a["D"], a["ql"],
                 a["kv"], a["qs"], a["MS"], S)

    assert call(o=0) == -1
    assert call(q=U) == -2
    assert call(D=256) == -3
    assert call(hq=5) == -4
    assert call(kv=0) == -6
    assert call(kv=17) == -6           # kv_len > max_seq_len
    assert call(qs=-1) == -6
    assert call(sc=0.0) == -9
    assert call(ql=0) == 0


def test_prefill_sched_checks(L):
    """grout_attn_prefill_sched: its counters are checked first, then the same
    argument checks as grout_attn_prefill (one shared validation path)."""
    f = L.grout_attn_prefill_sched
    ok = dict(q=A, k=A, v=A, o=A, sc=0.088, hq=4, hkv=2, D=128, ql=8, kv=8, qs=0, MS=16, c=A)

    def call(**kw):
        a = dict(ok, **kw)
        return f(a["q"], a["k"], a["v"], a["o"], a["sc"], a["hq"], a["hkv"], a["D"], a["ql"],
                 a["kv"], a["qs"], a["MS"], a["c"], S)

    assert call(c=0) == -1
    assert call(c=U) == -2
    assert call(o=0) == -1
    assert call(q=U) == -2
    assert call(D=256) == -3
    assert call(hq=5) == -4
    assert call(kv=17) == -6
    assert call(sc=0.0) == -9
    assert call(ql=0) == 0
    # 8 heavy and 8 light XCD queues and the exit counter, one 256-byte line each.
    assert L.grout_attn_prefill_sched_counter_bytes() == 17 * 256


def test_prefill_split_checks(L):
    f = L.grout_attn_prefill_split
    ok = dict(q=A, k=A, v=A, att=A, lse=A, sc=0.088, hq=8, hkv=2, D=128, ql=40, kv=40, qs=0,
              MS=64, bm=32, bn=32, gr=2, ns=3)

    def call(**kw):
        a = dict(ok, **kw)
        return f(a["q"], a["k"], a["v"], a["att"], a["lse"], a["sc"], a["hq"], a["hkv"], a["D"],
                 a["ql"], a["kv"], a["qs"], a["MS"], a["bm"], a["bn"], a["gr"], a["ns"], S)

    assert call(lse=0) == -1
    assert call(att=U) == -2
    assert call(D=64) == -3
    assert call(hq=7) == -4
    assert call(kv=65) == -6
    assert call(gr=3) == -7            # group must divide q_group_size (4)
    assert call(gr=0) == -7
    assert call(bm=48) == -9           # block_m a multiple of 32
    assert call(bm=16) == -9
    assert call(bn=0) == -8
    assert call(ns=0) == -8
    assert call(ns=1025) == -8
    assert call(ql=0) == 0
    mg = L.grout_attn_prefill_split_merge
    # att, lse, out, Hq, D, q_len, BM, group, NKS
    assert mg(A, A, 0, 8, 128, 40, 32, 2, 3, S) == -1
    assert mg(A, A, A, 8, 64, 40, 32, 2, 3, S) == -3
    assert mg(A, A, A, 8, 128, 40, 32, 3, 3, S) == -7
    assert mg(A, A, A, 8, 128, 40, 32, 2, 0, S) == -8
    assert mg(A, A, A, 8, 128, 0, 32, 2, 3, S) == 0
    # Scratch: ceil(40/32) * (8/2) tiles of 3 * 32 * 2 rows.
    rows = 2 * 4 * 3 * 32 * 2
    assert L.grout_attn_prefill_split_partial_bytes(8, 128, 40, 32, 2, 3) == rows * 128 * 2
    assert L.grout_attn_prefill_split_lse_bytes(8, 40, 32, 2, 3) == rows * 4
    assert L.grout_attn_prefill_split_lse_bytes(8, 40, 32, 3, 3) < 0


def test_decode_split_merge_checks(L):
    sp = L.grout_attn_decode_split
    # q, k, v, att, lse, scale, pos, hkv, G, D, MS, BN, NKS
    assert sp(A, A, A, A, A, 0x2DA8, 0, 8, 4, 128, 64, 32, 4, S) == -1
    assert sp(A, A, A, U, A, 0x2DA8, A, 8, 4, 128, 64, 32, 4, S) == -2
    assert sp(A, A, A, A, A, 0x2DA8, A, 8, 4, 64, 64, 32, 4, S) == -3
    assert sp(A, A, A, A, A, 0x2DA8, A, 8, 17, 128, 64, 32, 4, S) == -7
    assert sp(A, A, A, A, A, 0x2DA8, A, 8, 4, 128, 64, 0, 4, S) == -8
    assert sp(A, A, A, A, A, 0x2DA8, A, 8, 4, 128, 64, 32, 1025, S) == -8
    assert sp(A, A, A, A, A, 0x0000, A, 8, 4, 128, 64, 32, 4, S) == -9   # scale 0
    assert sp(A, A, A, A, A, 0x7C00, A, 8, 4, 128, 64, 32, 4, S) == -9   # scale inf
    mg = L.grout_attn_decode_merge
    assert mg(0, A, A, 8, 4, 128, 4, S) == -1
    assert mg(A, A, A, 8, 0, 128, 4, S) == -7
    assert mg(A, A, A, 8, 4, 128, 0, S) == -8


def test_decode_fused_checks(L):
    f = L.grout_attn_decode_fused
    base = [A] * 12 + [1e-6, 0x2DA8, 32, 8, 128, 64, 32, 4, 1, S]

    def call(i, v):
        a = list(base)
        a[i] = v
        return f(*a)

    assert f(*base[:10], 0, *base[11:]) == -1            # counters
    assert call(0, 0) == -1                               # qkv
    assert call(11, A + 2) == -2                          # position misaligned
    assert call(14, 30) == -4                             # heads
    assert call(16, 64) == -3                             # head_dim
    assert call(12, -1.0) == -9                           # eps


def test_decode_fused_noalloc_without_device(L):
    """With no usable device the set-up fails with the HIP error, and the
    failure is not kept: every later call tries again and reports its own
    status (here the same error), never a stored one."""
    import torch

    if torch.cuda.is_available():
        pytest.skip("a GPU is visible: the set-up would succeed")
    f = L.grout_attn_decode_fused_noalloc
    args = [A] * 9 + [1e-6, 0x2DA8, 32, 8, 128, 4200, 32, 16, 1, None]
    first = f(*args)
    assert first > 0, first                       # a hipError_t, not a validation code
    assert f(*args) == first
    # Validation still runs before the device is touched.
    bad = list(args)
    bad[16] = 0                                   # num_splits
    assert f(*bad) == -8
    bad = list(args)
    bad[12] = 256 * 3                             # num_kv_heads > 255, heads divisible
    bad[11] = 256 * 3
    assert f(*bad) == -11


def test_kv_cache_update_checks(L):
    f = L.grout_kv_cache_update_seq
    # new_k, new_v, k_cache, v_cache, start, S, Hkv, D, MS, stream
    assert f(0, A, A, A, 0, 4, 2, 128, 16, S) == -1
    assert f(A, A, A, A, 0, 4, 2, 126, 16, S) == -3       # head_dim not a multiple of 4
    assert f(A, A, A, A, 0, 4, 0, 128, 16, S) == -4
    assert f(A, A, A, A, 13, 4, 2, 128, 16, S) == -5      # 17 > max_seq_len
    assert f(A, A, A, A, -1, 4, 2, 128, 16, S) == -5
    assert f(A + 8, A, A, A, 0, 4, 2, 128, 16, S) == -2   # 8-byte aligned, 16-byte rows
    assert f(A, A, A, A, 0, 0, 2, 128, 16, S) == 0        # empty: nothing launched
    g = L.grout_kv_cache_update_seq_dynpos
    assert g(A, A, A, A, 0, 1, 2, 128, 16, S) == -1
    assert g(A, A, A, A, A + 2, 1, 2, 128, 16, S) == -2


def test_decode_layer_checks(L):
    f = L.grout_add_rms_norm_decode
    # residual, x, weight, out, residual_out, eps, n, stream
    assert f(A, 0, A, A, A, 1e-6, 5120, S) == -1
    assert f(A, A, A, U, A, 1e-6, 5120, S) == -2
    assert f(A, A, A, A, A, 1e-6, 0, S) == -9
    assert f(A, A, A, A, A, 1e-6, 5124, S) == -9          # not a multiple of 8
    assert f(A, A, A, A, A, 1e-6, 32776, S) == -9         # above the one-workgroup maximum
    assert f(A, A, A, A, A, -1.0, 5120, S) == -9
    g = L.grout_gemv_f16
    # weight, x, out, m, k, stream
    assert g(0, A, A, 8, 8, S) == -1
    assert g(A, A, 0, 8, 8, S) == -1
    assert g(U, A, A, 8, 8, S) == -2
    assert g(A, A, A + 1, 8, 8, S) == -2                  # out needs 2-byte alignment only
    assert g(A, A, A, 0, 8, S) == -9
    assert g(A, A, A, 8, 12, S) == -9
    assert g(A, A, A, 8, 32776, S) == -9
    assert L.grout_argmax_blocks(0) == -9
    assert L.grout_argmax_blocks((1 << 30) + 1) == -9
    assert [L.grout_argmax_blocks(n) for n in (1, 2048, 2049, 151936)] == [1, 1, 2, 75]
    a = L.grout_argmax_f16
    # logits, block_max, block_idx, token, n, stream
    assert a(0, A, A, A, 10, S) == -1
    assert a(A, A, 0, A, 10, S) == -1
    assert a(U, A, A, A, 10, S) == -2
    assert a(A, A + 2, A, A, 10, S) == -2
    assert a(A, A, A, A, 0, S) == -9


def test_token_step_op_checks(L):
    e = L.grout_embed_rms_norm_decode
    # token, table, vocab, weight, out, residual_out, eps, n, stream
    assert e(0, A, 10, A, A, A, 1e-6, 64, S) == -1
    assert e(A + 2, A, 10, A, A, A, 1e-6, 64, S) == -2    # token needs 4-byte alignment
    assert e(A, U, 10, A, A, A, 1e-6, 64, S) == -2
    assert e(A, A, 0, A, A, A, 1e-6, 64, S) == -9
    assert e(A, A, 10, A, A, A, 1e-6, 60, S) == -9
    s = L.grout_silu_mul_f16
    assert s(A, 0, A, 64, S) == -1
    assert s(A, A, U, 64, S) == -2
    assert s(A, A, A, 12, S) == -9
    assert s(A, A, A, 0, S) == -9
    gs = L.grout_gemv_silu_mul_f16
    # gate_up, x, out, n, k, stream
    assert gs(0, A, A, 8, 8, S) == -1
    assert gs(A, 0, A, 8, 8, S) == -1
    assert gs(A, A, 0, 8, 8, S) == -1
    assert gs(U, A, A, 8, 8, S) == -2
    assert gs(A, A, A + 1, 8, 8, S) == -2                 # out needs 2-byte alignment only
    assert gs(A, A, A, 0, 8, S) == -9
    assert gs(A, A, A, (1 << 29) + 1, 8, S) == -9
    assert gs(A, A, A, 8, 12, S) == -9
    assert gs(A, A, A, 8, 32776, S) == -9


def test_cast_checks(L):
    c = L.grout_cast_to_f16
    # src, dtype, dst, n, stream
    assert c(0, 1, A, 8, S) == -1
    assert c(A, 1, U, 8, S) == -2
    assert c(A, 4, A, 8, S) == -9
    assert c(A, -1, A, 8, S) == -9
    assert c(A, 1, A, -1, S) == -9
    assert c(A, 1, A, 0, S) == 0        # nothing to convert: no launch


def _qwen3_model(**over):
    import ctypes

    from grout_amd import _lib

    layers = (_lib.Qwen3Layer * 2)(*[_lib.Qwen3Layer(*([A] * 10)) for _ in range(2)])
    kw = dict(num_layers=2, hidden=256, intermediate=512, vocab=1000, num_q_heads=4,
              num_kv_heads=2, head_dim=128, max_seq_len=64, block_n=32, num_splits=3,
              eps=1e-6, qk_scale_f16=0x2DA8, layers=layers, embed_tokens=A, final_norm=A,
              lm_head=A, inv_freq=A, token=A, d_position=A, logits=A, workspace=A)
    kw.update(over)
    m = _lib.Qwen3Model(**kw)
    m._keep = layers
    return ctypes.byref(m)


def test_token_step_runner_checks(L):
    import ctypes

    from grout_amd import _lib

    ws = L.grout_qwen3_workspace_bytes
    assert ws(None) == -1
    n = ws(_qwen3_model())
    # hidden x3 + qkv + q_out + attn_out + attn_proj + ff + ff_down
    # + partials + lse + counters + argmax blocks, each rounded up to 256 bytes.
    assert n > 2 * (3 * 256 + 8 * 128 + 6 * 128 + 4 * 128 + 256 + 1024 + 512 + 256)
    assert n % 256 == 0
    assert ws(_qwen3_model(num_layers=0)) == -9
    assert ws(_qwen3_model(head_dim=64)) == -3
    assert ws(_qwen3_model(num_q_heads=5)) == -4
    assert ws(_qwen3_model(hidden=260)) == -9
    assert ws(_qwen3_model(num_splits=0)) == -8
    assert ws(_qwen3_model(layers=None)) == -1
    st = L.grout_qwen3_decode_step
    assert st(_qwen3_model(workspace=None), S) == -1
    assert st(_qwen3_model(workspace=A + 16), S) == -2      # workspace needs 256-byte alignment
    h = ctypes.c_void_p()
    assert L.grout_qwen3_runner_create(_qwen3_model(), 0, S, ctypes.byref(h)) == -10  # null stream
    assert L.grout_qwen3_runner_create(_qwen3_model(), 64, A, ctypes.byref(h)) == -5
    assert L.grout_qwen3_runner_step(None, 0, None) == -10
    assert L.grout_qwen3_runner_run(None, 0, 1) == -10
    assert L.grout_qwen3_runner_seed_token(None, 0) == -10
    assert L.grout_qwen3_runner_destroy(None) == 0
    assert _lib.SIGNATURES["grout_qwen3_runner_create"][0] is ctypes.c_int32


def test_graph_handle_checks(L):
    assert L.grout_graph_begin(None) == -10
    assert L.grout_graph_launch(None, None) == -10
    assert L.grout_graph_destroy(None) == 0
    assert L.grout_set_position_async(None, 3, None) == -1
    assert L.grout_decode_runner_step(None, 0) == -10
    assert L.grout_decode_runner_run(None, 0, 4) == -10
    assert L.grout_decode_runner_destroy(None) == 0


def test_inv_freq_matches_oracle(L):
    import ctypes

    for theta in (1e4, 1e6, 5e5):
        out = (ctypes.c_float * 64)()
        assert L.grout_build_inv_freq(theta, 128, out) == 0
        got = np.array(list(out), dtype=np.float32)
        assert np.array_equal(got, oracle.build_inv_freq(theta))
    out = (ctypes.c_float * 64)()
    assert L.grout_build_inv_freq(1e6, 127, out) == -3
    assert L.grout_build_inv_freq(-1.0, 128, out) == -9


def test_scratch_sizes(L):
    assert L.grout_attn_decode_partial_bytes(8, 8, 128, 32) == 8 * 32 * 8 * 128 * 2
    assert L.grout_attn_decode_lse_bytes(8, 8, 32) == 8 * 32 * 8 * 4
    assert L.grout_attn_decode_counter_bytes(8) >= 9 * 4
    assert L.grout_attn_decode_partial_bytes(0, 8, 128, 32) < 0


def test_pick_splits(L):
    f = L.grout_attn_decode_pick_splits
    # One workgroup per CU at long context: Hkv * NKS covers the CUs.
    assert f(256, 8, 32768 + 1024, 32) * 8 >= 256
    # Short contexts do not get splits shorter than one 64-token chunk.
    assert f(256, 8, 64, 32) == 1
    assert f(256, 8, 4097, 32) <= (4097 + 63) // 64
    assert f(0, 8, 32768, 32) >= 1
    for ctx in (1, 100, 4097, 33792, 10 ** 6):
        assert 1 <= f(256, 8, ctx, 32) <= 1024


def test_pick_splits_grouped(L):
    f, g = L.grout_attn_decode_pick_splits, L.grout_attn_decode_pick_splits_grouped
    # group 1 is the ungrouped count, at every context and head count.
    for hkv in (1, 2, 4, 8, 16):
        for ctx in (1, 100, 4097, 33792, 10 ** 6):
            assert g(256, hkv, 1, ctx, 32) == f(256, hkv, ctx, 32)
    # NS * G within one 512-row merge batch leaves the count alone.
    assert g(256, 8, 8, 32768, 32) == 32         # Qwen3-32B
    assert g(256, 8, 4, 32768, 32) == 32         # Qwen3-4B
    assert g(256, 4, 8, 32768, 32) == 64         # 32 Q / 4 KV heads: 64 x 8 = 512
    # Beyond one batch it takes the batch's split count while that keeps half the CUs.
    assert g(256, 4, 16, 32768, 32) == 32        # 64 Q / 4 KV heads
    assert g(256, 4, 12, 32768, 32) == 42        # 512 // 12
    assert g(256, 2, 16, 32768, 32) == 64        # half the CUs: 128 / 2 KV heads
    # Short contexts still get no split shorter than one 64-token chunk.
    assert g(256, 4, 16, 1000, 32) == (1000 + 63) // 64
    assert g(256, 4, 0, 32768, 32) == f(256, 4, 32768, 32)   # group <= 0 reads as 1


def test_python_mirror_shape_errors():
    torch = pytest.importorskip("torch")
    import grout_amd

    h = torch.float16
    q = torch.zeros((4, 8, 128), dtype=h)
    k = torch.zeros((4, 2, 128), dtype=h)
    bad_v = torch.zeros((3, 2, 128), dtype=h)
    w = torch.ones(128, dtype=h)
    inv = torch.ones(64)
    cache = torch.zeros((2, 16, 128), dtype=h)
    with pytest.raises(grout_amd.GroutError, match="v shape mismatch"):
        grout_amd.qk_norm_rope_kv_prefill(q, k, bad_v, w, w, inv, torch.zeros_like(q), cache,
                                          cache, 1e-6, 0)
    with pytest.raises(grout_amd.GroutError, match="exceeds max_seq_len"):
        grout_amd.qk_norm_rope_kv_prefill(q, k, k, w, w, inv, torch.zeros_like(q), cache, cache,
                                          1e-6, 13)
    with pytest.raises(grout_amd.GroutError, match="attend output shape mismatch"):
        grout_amd.attend_prefill(q, cache, cache, torch.zeros((4, 4, 128), dtype=h), 0)
    with pytest.raises(grout_amd.GroutError, match="rank 3"):
        grout_amd.attend_prefill(q[0], cache, cache, q[0], 0)
    wm = torch.zeros((16, 64), dtype=h)
    with pytest.raises(grout_amd.GroutError, match="x must have 64 elements"):
        grout_amd.gemv_f16(wm, torch.zeros(32, dtype=h), torch.zeros(16, dtype=h))
    with pytest.raises(grout_amd.GroutError, match="out must have 16 elements"):
        grout_amd.gemv_f16(wm, torch.zeros(64, dtype=h), torch.zeros(15, dtype=h))
    lay = {"input_norm": torch.zeros(256, dtype=h), "qkv_proj": torch.zeros((1024, 256), dtype=h),
           "q_norm": torch.zeros(128, dtype=h), "k_norm": torch.zeros(128, dtype=h),
           "o_proj": torch.zeros((256, 512), dtype=h), "post_attn_norm": torch.zeros(256, dtype=h),
           "gate_up_proj": torch.zeros((1024, 256), dtype=h),
           "down_proj": torch.zeros((256, 512), dtype=h),
           "k_cache": torch.zeros((2, 16, 128), dtype=h), "v_cache": torch.zeros((2, 16, 128), dtype=h)}
    kw = dict(embed_tokens=torch.zeros((10, 256), dtype=h), final_norm=torch.zeros(256, dtype=h),
              lm_head=torch.zeros((10, 256), dtype=h), inv_freq=torch.zeros(64),
              token=torch.zeros(1, dtype=torch.int32), position=torch.zeros(1, dtype=torch.int32),
              logits=torch.zeros(10, dtype=h), num_q_heads=4, num_kv_heads=2, eps=1e-6,
              qk_scale_f16_bits=0x2DA8)
    with pytest.raises(grout_amd.GroutError, match="o_proj shape"):
        grout_amd.Qwen3DecodeRunner(layers=[dict(lay, o_proj=torch.zeros((256, 256), dtype=h))],
                                    **kw)
    with pytest.raises(grout_amd.GroutError, match="lm_head must be"):
        grout_amd.Qwen3DecodeRunner(layers=[lay], **dict(kw, lm_head=torch.zeros((9, 256), dtype=h)))
    with pytest.raises(grout_amd.GroutError, match="must be a device tensor"):
        grout_amd.Qwen3DecodeRunner(layers=[lay], **kw)   # CPU tensors
    with pytest.raises(grout_amd.GroutError, match="weight must have 64 elements"):
        z = torch.zeros(64, dtype=h)
        grout_amd.add_rms_norm_decode(z, z, torch.zeros(32, dtype=h), z, z, 1e-6)
