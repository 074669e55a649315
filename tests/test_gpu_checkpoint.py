"""GPU parity of the checkpoint path (src/loader.rs:107-145 cast_to_f16,
src/model.rs:1373-1470 weight layout) against the oracle: the device element
conversion bit-exact for every dtype (NaN stays NaN), every loaded tensor
bit-exact against the oracle's conversion of the same file bytes, q/k/v and
gate/up merged in the reference's row order, tied embeddings shared, and a
decode token step run from the loaded checkpoint matching the oracle's step
on the same converted weights."""
import numpy as np
import pytest

import oracle
from tests._util import assert_close_attn, raw_bytes, write_qwen3_checkpoint

pytestmark = pytest.mark.gpu


def _cast_gpu(torch, raw: np.ndarray, dtype: str, n: int, offset: int = 0):
    import grout_amd
    from grout_amd.checkpoint import DTYPE_CODES

    src = torch.from_numpy(np.ascontiguousarray(raw).view(np.uint8)).cuda()
    dst = torch.full((n + offset + 16,), 7.0, dtype=torch.float16, device="cuda")
    grout_amd._check(grout_amd.lib().grout_cast_to_f16(
        src.data_ptr(), DTYPE_CODES[dtype], dst[offset:].data_ptr(), n,
        torch.cuda.current_stream().cuda_stream), "cast")
    torch.cuda.synchronize()
    out = dst.cpu().numpy()
    assert np.all(out[:offset] == 7.0) and np.all(out[offset + n:] == 7.0), "write outside dst"
    return out[offset:offset + n]


def _same(a, b):
    nan = np.isnan(b)
    assert np.array_equal(np.isnan(a), nan)
    assert np.array_equal(a[~nan].view(np.uint16), b[~nan].view(np.uint16))


def test_cast_all_dtypes_match_oracle(gpu):
    import torch

    g = np.random.default_rng(11)
    allbits = np.arange(65536, dtype=np.uint16)
    _same(_cast_gpu(torch, allbits, "BF16", 65536), oracle.cast_to_f16(allbits, "BF16"))
    _same(_cast_gpu(torch, allbits, "F16", 65536), allbits.view(np.float16))
    x = np.concatenate([g.standard_normal(100000) * 3000, g.standard_normal(5000) * 1e-6,
                        [0.0, -0.0, 65504.0, 65519.996, 65520.0, 1e30, -np.inf, np.nan,
                         2.0 ** -25, 2.0 ** -25 * (1 + 2.0 ** -20), 3 * 2.0 ** -26,
                         1 + 2.0 ** -11 + 2.0 ** -40]])
    for dtype, arr in (("F32", x.astype(np.float32)), ("F64", x)):
        _same(_cast_gpu(torch, arr, dtype, x.size), oracle.cast_to_f16(arr, dtype))
    # Ragged n (scalar tail) into a row range that starts mid-buffer.
    bits = g.integers(0, 65536, 1003, dtype=np.uint16)
    _same(_cast_gpu(torch, bits, "BF16", 1003, offset=8), oracle.cast_to_f16(bits, "BF16"))


def _oracle_model(tensors, cfg, max_seq):
    def conv(name):
        dtype, t = tensors[name]
        return oracle.cast_to_f16(raw_bytes(t), dtype).reshape(tuple(t.shape))

    hkv = cfg.num_key_value_heads
    m = {"num_q_heads": cfg.num_attention_heads, "num_kv_heads": hkv, "eps": cfg.rms_norm_eps,
         "qk_scale_f16_bits": oracle.f16_bits(1.0 / np.sqrt(128.0)), "layers": [],
         "embed_tokens": conv("model.embed_tokens.weight"),
         "final_norm": conv("model.norm.weight"),
         "inv_freq": oracle.build_inv_freq(cfg.rope_theta)}
    m["lm_head"] = m["embed_tokens"] if cfg.tie_word_embeddings else conv("lm_head.weight")
    for i in range(cfg.num_hidden_layers):
        p = f"model.layers.{i}."
        m["layers"].append({
            "input_norm": conv(p + "input_layernorm.weight"),
            "qkv_proj": np.concatenate([conv(p + "self_attn.q_proj.weight"),
                                        conv(p + "self_attn.k_proj.weight"),
                                        conv(p + "self_attn.v_proj.weight")]),
            "q_norm": conv(p + "self_attn.q_norm.weight"),
            "k_norm": conv(p + "self_attn.k_norm.weight"),
            "o_proj": conv(p + "self_attn.o_proj.weight"),
            "post_attn_norm": conv(p + "post_attention_layernorm.weight"),
            "gate_up_proj": np.concatenate([conv(p + "mlp.gate_proj.weight"),
                                            conv(p + "mlp.up_proj.weight")]),
            "down_proj": conv(p + "mlp.down_proj.weight"),
            "k_cache": np.zeros((hkv, max_seq, 128), np.float16),
            "v_cache": np.zeros((hkv, max_seq, 128), np.float16)})
    return m


@pytest.mark.parametrize("tie", [False, True])
def test_load_qwen3_matches_oracle(gpu, tmp_path, tie):
    from grout_amd.checkpoint import load_qwen3

    tensors = write_qwen3_checkpoint(str(tmp_path), 20 + tie, tie=tie)
    dev = load_qwen3(str(tmp_path), max_seq_len=32)
    cfg = dev["config"]
    ref = _oracle_model(tensors, cfg, 32)
    for key in ("embed_tokens", "final_norm", "lm_head"):
        assert np.array_equal(dev[key].cpu().numpy().view(np.uint16), ref[key].view(np.uint16)), key
    if tie:
        assert dev["lm_head"].data_ptr() == dev["embed_tokens"].data_ptr()
    assert np.array_equal(dev["inv_freq"].cpu().numpy(), ref["inv_freq"])
    for i, (L, R) in enumerate(zip(dev["layers"], ref["layers"])):
        for key, v in R.items():
            got = L[key].cpu().numpy()
            assert got.shape == v.shape, (i, key)
            assert np.array_equal(got.view(np.uint16), v.view(np.uint16)), (i, key)
    # Row order of the merged projections: Q rows first, then K, then V.
    k = oracle.cast_to_f16(raw_bytes(tensors["model.layers.1.self_attn.k_proj.weight"][1]), "BF16")
    assert np.array_equal(dev["layers"][1]["qkv_proj"][4 * 128].cpu().numpy(), k[:256])


def test_token_step_from_checkpoint(gpu, tmp_path):
    import torch
    import grout_amd
    from grout_amd.checkpoint import load_qwen3

    tensors = write_qwen3_checkpoint(str(tmp_path), 30)
    dev = load_qwen3(str(tmp_path), max_seq_len=32)
    cfg = dev["config"]
    ref = _oracle_model(tensors, cfg, 32)
    token = torch.tensor([42], dtype=torch.int32, device="cuda")
    position = torch.zeros((1,), dtype=torch.int32, device="cuda")
    logits = torch.zeros((cfg.vocab_size,), dtype=torch.float16, device="cuda")
    runner = grout_amd.Qwen3DecodeRunner(
        layers=dev["layers"], embed_tokens=dev["embed_tokens"], final_norm=dev["final_norm"],
        lm_head=dev["lm_head"], inv_freq=dev["inv_freq"], token=token, position=position,
        logits=logits, num_q_heads=cfg.num_attention_heads,
        num_kv_heads=cfg.num_key_value_heads, eps=cfg.rms_norm_eps,
        qk_scale_f16_bits=ref["qk_scale_f16_bits"], num_splits=2, block_n=32, prime_position=0)
    try:
        torch.cuda.synchronize()
        tok = 42
        for pos in range(4):
            if pos:
                runner.step(pos)
            rl, _ = oracle.qwen3_decode_step(ref, tok, pos, 32, 2, fused_ranges=True)
            gl = logits.cpu().numpy()
            assert_close_attn(gl, rl, f"position {pos} logits", atol=1e-2, rtol=1e-2)
            tok = int(token.item())
            assert tok == oracle.argmax_f16(gl)
    finally:
        runner.close()
