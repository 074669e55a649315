"""CPU tests of the checkpoint formats (src/config.rs:7-38, src/loader.rs:21-145):
config parsing, the shard index, safetensors header parsing against the bytes
the safetensors library wrote, name and dtype errors, and the oracle's element
conversion (cast_to_f16) against numpy for every dtype."""
import json
import os

import numpy as np
import pytest

import oracle
from tests._util import raw_bytes, write_qwen3_checkpoint


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    pytest.importorskip("safetensors")
    d = str(tmp_path_factory.mktemp("qwen3_ckpt"))
    return d, write_qwen3_checkpoint(d, 10)


def test_config_parse(ckpt):
    from grout_amd.checkpoint import Qwen3Config

    cfg = Qwen3Config.from_model_dir(ckpt[0])
    assert (cfg.vocab_size, cfg.hidden_size, cfg.intermediate_size, cfg.num_hidden_layers) == \
        (1000, 256, 512, 2)
    assert (cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim) == (4, 2, 128)
    assert cfg.num_kv_groups() == 2
    assert cfg.rms_norm_eps == np.float32(1e-6) and cfg.rope_theta == 1e6
    assert cfg.tie_word_embeddings is False and cfg.eos_token_id == 151645


def test_config_errors(tmp_path):
    import grout_amd
    from grout_amd.checkpoint import Qwen3Config

    with pytest.raises(grout_amd.GroutError, match="failed to read"):
        Qwen3Config.from_model_dir(str(tmp_path))
    (tmp_path / "config.json").write_text("{not json")
    with pytest.raises(grout_amd.GroutError, match="failed to parse"):
        Qwen3Config.from_model_dir(str(tmp_path))
    base = {"vocab_size": 10, "hidden_size": 8, "intermediate_size": 8, "num_hidden_layers": 1,
            "num_attention_heads": 2, "num_key_value_heads": 1, "head_dim": 128,
            "rms_norm_eps": 1e-6, "rope_theta": 1e6, "max_position_embeddings": 64,
            "tie_word_embeddings": True, "use_sliding_window": False, "eos_token_id": 3}
    assert Qwen3Config.from_dict(dict(base, extra_key=[1, 2])).vocab_size == 10
    with pytest.raises(grout_amd.GroutError, match="missing field `head_dim`"):
        Qwen3Config.from_dict({k: v for k, v in base.items() if k != "head_dim"})
    with pytest.raises(grout_amd.GroutError, match="eos_token_id"):
        Qwen3Config.from_dict(dict(base, eos_token_id=[1, 2]))   # a list is not a u32
    with pytest.raises(grout_amd.GroutError, match="tie_word_embeddings"):
        Qwen3Config.from_dict(dict(base, tie_word_embeddings=1))


def test_safetensors_headers_match_writer(ckpt):
    from grout_amd.checkpoint import WeightLoader

    d, tensors = ckpt
    ld = WeightLoader(d)
    try:
        assert set(ld.weight_map) == set(tensors)
        assert len(ld.shards) == 2
        for name, (dtype, t) in tensors.items():
            got_dtype, shape = ld.info(name)
            assert got_dtype == dtype and shape == list(t.shape), name
            assert np.array_equal(np.frombuffer(ld.raw(name), np.uint8), raw_bytes(t)), name
    finally:
        ld.close()


def test_loader_errors(ckpt, tmp_path):
    import grout_amd
    from grout_amd.checkpoint import SafetensorsFile, WeightLoader

    with pytest.raises(grout_amd.GroutError, match="index.json"):
        WeightLoader(str(tmp_path))
    ld = WeightLoader(ckpt[0])
    try:
        with pytest.raises(grout_amd.GroutError, match="not found in index"):
            ld.info("model.layers.9.mlp.up_proj.weight")
    finally:
        ld.close()
    bad = tmp_path / "bad.safetensors"
    hdr = json.dumps({"x": {"dtype": "BF16", "shape": [4], "data_offsets": [0, 6]}}).encode()
    bad.write_bytes(len(hdr).to_bytes(8, "little") + hdr + bytes(8))
    with pytest.raises(grout_amd.GroutError, match="do not match"):
        SafetensorsFile(str(bad))
    odd = tmp_path / "odd.safetensors"
    hdr = json.dumps({"x": {"dtype": "BF16", "shape": [4]}}).encode()   # no data_offsets
    odd.write_bytes(len(hdr).to_bytes(8, "little") + hdr + bytes(8))
    with pytest.raises(grout_amd.GroutError, match="bad header entry"):
        SafetensorsFile(str(odd))
    empty = tmp_path / "empty.safetensors"
    empty.write_bytes(b"")
    with pytest.raises(grout_amd.GroutError, match="failed to map"):
        SafetensorsFile(str(empty))
    trunc = tmp_path / "trunc.safetensors"
    trunc.write_bytes((1 << 40).to_bytes(8, "little") + b"{}")
    with pytest.raises(grout_amd.GroutError, match="past the end"):
        SafetensorsFile(str(trunc))


def test_cast_to_f16_oracle_against_numpy():
    """src/loader.rs:107-145 element rules, pinned on numpy's conversions."""
    g = np.random.default_rng(5)
    allbits = np.arange(65536, dtype=np.uint16)
    f32 = (allbits.astype(np.uint32) << 16).view(np.float32)
    with np.errstate(over="ignore", invalid="ignore"):
        exp = f32.astype(np.float16)
    got = oracle.cast_to_f16(allbits, "BF16")
    nan = np.isnan(f32)
    assert np.array_equal(got[~nan].view(np.uint16), exp[~nan].view(np.uint16))
    assert np.all(np.isnan(got[nan]))
    x = np.concatenate([g.standard_normal(50000) * 3000, g.standard_normal(5000) * 1e-6,
                        [0.0, -0.0, 65504.0, 65519.996, 65520.0, 1e30, -np.inf, 2.0 ** -25,
                         2.0 ** -25 * (1 + 2.0 ** -20), 3 * 2.0 ** -26]])
    with np.errstate(over="ignore"):
        assert np.array_equal(oracle.cast_to_f16(x.astype(np.float32), "F32").view(np.uint16),
                              x.astype(np.float32).astype(np.float16).view(np.uint16))
        # F64 goes through f32 (`x as f32`): double rounding, as the reference.
        assert np.array_equal(oracle.cast_to_f16(x, "F64").view(np.uint16),
                              x.astype(np.float32).astype(np.float16).view(np.uint16))
    h = g.integers(0, 65536, 1000, dtype=np.uint16)
    assert np.array_equal(oracle.cast_to_f16(h, "F16").view(np.uint16), h)
    # A value that rounds differently through f32 than directly: 1 + 2^-11 + 2^-40
    # is above the f16 tie point but rounds to the tie in f32, then to even.
    v = np.array([1 + 2.0 ** -11 + 2.0 ** -40])
    assert oracle.cast_to_f16(v, "F64")[0] == np.float16(1.0)
    with pytest.raises(ValueError):
        oracle.cast_to_f16(h, "I8")
