"""Qwen3 checkpoint formats for the decode path.

* :class:`Qwen3Config` — ``config.json`` (``Qwen3Config``, src/config.rs:7-38);
* :class:`SafetensorsFile` / :class:`WeightLoader` — the sharded safetensors
  checkpoint behind ``model.safetensors.index.json`` (``WeightLoader``,
  src/loader.rs:21-104), memory-mapped, headers parsed here (JSON only; nothing
  in a file is executed);
* :func:`load_qwen3` — the model constructor's weight layout
  (src/model.rs:1373-1470): embedding, lm_head (tied or not), final norm, and
  per layer the merged ``qkv_proj`` (rows Q | K | V) and ``gate_up_proj``
  (rows gate | up), norms, ``o_proj``, ``down_proj`` and zeroed KV caches.

Element conversion runs on the GPU: the raw bytes of a tensor are copied to
the device once and ``grout_cast_to_f16`` writes f16 straight into the
destination (a row range of a merged matrix where the reference concatenates,
src/model.rs:6021-6070), instead of the reference's per-element host loop
(cast_to_f16, src/loader.rs:107-145).
"""
from __future__ import annotations

import dataclasses
import json
import mmap
import os
import struct
import warnings

from . import GroutError, _check, _ensure, _stream, build_inv_freq, lib

DTYPE_CODES = {"F16": 0, "BF16": 1, "F32": 2, "F64": 3}
DTYPE_WIDTH = {"F16": 2, "BF16": 2, "F32": 4, "F64": 8, "I8": 1, "U8": 1, "I16": 2, "U16": 2,
               "I32": 4, "U32": 4, "I64": 8, "U64": 8, "BOOL": 1, "F8_E4M3": 1, "F8_E5M2": 1}


@dataclasses.dataclass
class Qwen3Config:
    """src/config.rs:7-21; unknown keys of config.json are ignored (serde's default)."""
    vocab_size: int
    hidden_size: int
    intermediate_size: int
    num_hidden_layers: int
    num_attention_heads: int
    num_key_value_heads: int
    head_dim: int
    rms_norm_eps: float
    rope_theta: float
    max_position_embeddings: int
    tie_word_embeddings: bool
    use_sliding_window: bool
    eos_token_id: int

    @classmethod
    def from_dict(cls, d: dict) -> "Qwen3Config":
        kw = {}
        for f in dataclasses.fields(cls):
            if f.name not in d:
                raise GroutError(f"config.json: missing field `{f.name}`")
            v = d[f.name]
            if f.type == "bool":
                _ensure(isinstance(v, bool), f"config.json: `{f.name}` must be a bool")
            elif f.type == "int":
                _ensure(isinstance(v, int) and not isinstance(v, bool) and v >= 0,
                        f"config.json: `{f.name}` must be an unsigned integer")
            else:
                _ensure(isinstance(v, (int, float)) and not isinstance(v, bool),
                        f"config.json: `{f.name}` must be a number")
                v = float(struct.unpack("<f", struct.pack("<f", float(v)))[0])  # serde's f32
            kw[f.name] = v
        return cls(**kw)

    @classmethod
    def from_model_dir(cls, model_dir: str) -> "Qwen3Config":
        """src/config.rs:24-33."""
        path = os.path.join(model_dir, "config.json")
        try:
            with open(path) as fh:
                text = fh.read()
        except OSError as e:
            raise GroutError(f"failed to read {path}: {e}") from e
        try:
            d = json.loads(text)
        except json.JSONDecodeError as e:
            raise GroutError(f"failed to parse {path}: {e}") from e
        return cls.from_dict(d)

    def num_kv_groups(self) -> int:
        return self.num_attention_heads // self.num_key_value_heads


class SafetensorsFile:
    """One memory-mapped safetensors file: an 8-byte little-endian header size,
    a JSON header {name: {dtype, shape, data_offsets}}, then the data."""

    def __init__(self, path: str):
        self.path = path
        try:
            with open(path, "rb") as fh:
                self._mm = mmap.mmap(fh.fileno(), 0, access=mmap.ACCESS_READ)
        except (OSError, ValueError) as e:  # missing, unreadable or empty file
            raise GroutError(f"failed to map {path}: {e}") from e
        size = len(self._mm)
        _ensure(size >= 8, f"{path}: not a safetensors file")
        (n,) = struct.unpack("<Q", self._mm[:8])
        _ensure(8 + n <= size, f"{path}: header size {n} past the end of the file")
        try:
            header = json.loads(bytes(self._mm[8:8 + n]))
        except (json.JSONDecodeError, UnicodeDecodeError) as e:
            raise GroutError(f"{path}: bad header: {e}") from e
        _ensure(isinstance(header, dict), f"{path}: bad header: not a JSON object")
        self.data_start = 8 + n
        self.metadata = header.pop("__metadata__", None)
        self.tensors = {}
        for name, info in header.items():
            try:
                dtype, shape = info["dtype"], [int(x) for x in info["shape"]]
                b, e = (int(x) for x in info["data_offsets"])
            except (KeyError, TypeError, ValueError) as err:
                raise GroutError(f"{path}: bad header entry `{name}`: {err!r}") from err
            count = 1
            for s in shape:
                count *= s
            width = DTYPE_WIDTH.get(dtype)
            _ensure(width is not None, f"{path}: `{name}` has unknown dtype {dtype}")
            _ensure(0 <= b <= e and self.data_start + e <= size and e - b == count * width,
                    f"{path}: `{name}` data_offsets {b}..{e} do not match {dtype}{shape}")
            self.tensors[name] = (dtype, shape, b, e)

    def raw(self, name: str) -> memoryview:
        """The tensor's bytes, a view of the mapping (no copy)."""
        _, _, b, e = self.tensors[name]
        return memoryview(self._mm)[self.data_start + b:self.data_start + e]

    def close(self):
        self._mm.close()


class WeightLoader:
    """src/loader.rs:21-104: the shard index, every shard memory-mapped once."""

    def __init__(self, model_dir: str):
        self.model_dir = model_dir
        index_path = os.path.join(model_dir, "model.safetensors.index.json")
        try:
            with open(index_path) as fh:
                index = json.load(fh)
        except OSError as e:
            raise GroutError(f"failed to read {index_path}: {e}") from e
        except json.JSONDecodeError as e:
            raise GroutError(f"failed to parse {index_path}: {e}") from e
        _ensure(isinstance(index.get("weight_map"), dict), f"{index_path}: no weight_map")
        self.weight_map = dict(index["weight_map"])
        self.shards = {s: SafetensorsFile(os.path.join(model_dir, s))
                       for s in sorted(set(self.weight_map.values()))}
        self._staging = None

    def _entry(self, name: str):
        shard = self.weight_map.get(name)
        if shard is None:
            raise GroutError(f"tensor `{name}` not found in index")
        f = self.shards[shard]
        if name not in f.tensors:
            raise GroutError(f"tensor `{name}` not found in `{shard}`")
        return f

    def info(self, name: str):
        """(dtype, shape) of a tensor."""
        dtype, shape, _, _ = self._entry(name).tensors[name]
        return dtype, list(shape)

    def raw(self, name: str) -> memoryview:
        return self._entry(name).raw(name)

    def load_into(self, name: str, out) -> None:
        """Convert tensor `name` to f16 into the device tensor `out` (a contiguous
        f16 view with the tensor's element count, e.g. a row range)."""
        import torch

        dtype, shape = self.info(name)
        code = DTYPE_CODES.get(dtype)
        if code is None:
            raise GroutError(f"failed to cast `{name}` from {dtype}: unsupported dtype for fp16 cast")
        count = 1
        for s in shape:
            count *= s
        _ensure(out.dtype == torch.float16 and out.is_cuda and out.is_contiguous(),
                f"`{name}`: destination must be a contiguous device f16 tensor")
        _ensure(out.numel() == count, f"`{name}`: {count} elements into a view of {out.numel()}")
        raw = self.raw(name)
        nbytes = len(raw)
        if count == 0:
            return
        if self._staging is None or self._staging.numel() < nbytes:
            self._staging = torch.empty((max(nbytes, 1 << 20),), dtype=torch.uint8,
                                        device=out.device)
        with warnings.catch_warnings():  # the mapping is read-only; torch only reads it
            warnings.simplefilter("ignore", UserWarning)
            host = torch.frombuffer(raw, dtype=torch.uint8, count=nbytes)
        stage = self._staging[:nbytes]
        stage.copy_(host)
        _check(lib().grout_cast_to_f16(stage.data_ptr(), code, out.data_ptr(), count, _stream()),
               f"cast_to_f16 `{name}`")

    def load_device_f16(self, name: str, device="cuda"):
        """load_device_f16 (src/loader.rs:86-100): a new device f16 tensor of the
        tensor's shape."""
        import torch

        _, shape = self.info(name)
        out = torch.empty(shape, dtype=torch.float16, device=device)
        self.load_into(name, out)
        return out

    def load_rows(self, names, device="cuda"):
        """concat_weight_rows_2d (src/model.rs:6021-6070) of rank-2 tensors with
        equal column counts, converted straight into their row ranges."""
        import torch

        _ensure(len(names) > 0, "concat_weight_rows_2d requires at least one tensor")
        shapes = [self.info(n)[1] for n in names]
        for n, s in zip(names, shapes):
            _ensure(len(s) == 2, f"concat_weight_rows_2d expects rank-2 tensors, got {s} ({n})")
            _ensure(s[1] == shapes[0][1],
                    f"concat_weight_rows_2d: mismatched columns {s[1]} vs {shapes[0][1]}")
        rows = sum(s[0] for s in shapes)
        out = torch.empty((rows, shapes[0][1]), dtype=torch.float16, device=device)
        r = 0
        for n, s in zip(names, shapes):
            self.load_into(n, out[r:r + s[0]])
            r += s[0]
        return out

    def close(self):
        for f in self.shards.values():
            f.close()
        self._staging = None


def load_qwen3(model_dir: str, max_seq_len: int, device="cuda") -> dict:
    """The weights of Qwen3Model's constructor (src/model.rs:1373-1470) on the
    device, in the layout :class:`grout_amd.Qwen3DecodeRunner` takes:
    returns {config, layers, embed_tokens, final_norm, lm_head, inv_freq}."""
    import torch

    cfg = Qwen3Config.from_model_dir(model_dir)
    _ensure(cfg.head_dim == 128, f"head_dim {cfg.head_dim}: the attention kernels need 128")
    _ensure(cfg.num_key_value_heads > 0 and
            cfg.num_attention_heads % cfg.num_key_value_heads == 0,
            "num_attention_heads must be a multiple of num_key_value_heads")
    _ensure(max_seq_len >= 1, "max_seq_len must be positive")
    ld = WeightLoader(model_dir)
    try:
        embed = ld.load_device_f16("model.embed_tokens.weight", device)
        lm_head = embed if cfg.tie_word_embeddings else ld.load_device_f16("lm_head.weight",
                                                                            device)
        norm = ld.load_device_f16("model.norm.weight", device)
        layers = []
        hkv, d = cfg.num_key_value_heads, cfg.head_dim
        for i in range(cfg.num_hidden_layers):
            p = f"model.layers.{i}."

            def one(suffix):
                return ld.load_device_f16(p + suffix, device)

            layers.append({
                "input_norm": one("input_layernorm.weight"),
                "qkv_proj": ld.load_rows([p + "self_attn.q_proj.weight",
                                          p + "self_attn.k_proj.weight",
                                          p + "self_attn.v_proj.weight"], device),
                "q_norm": one("self_attn.q_norm.weight"),
                "k_norm": one("self_attn.k_norm.weight"),
                "o_proj": one("self_attn.o_proj.weight"),
                "post_attn_norm": one("post_attention_layernorm.weight"),
                "gate_up_proj": ld.load_rows([p + "mlp.gate_proj.weight",
                                              p + "mlp.up_proj.weight"], device),
                "down_proj": one("mlp.down_proj.weight"),
                "k_cache": torch.zeros((hkv, max_seq_len, d), dtype=torch.float16, device=device),
                "v_cache": torch.zeros((hkv, max_seq_len, d), dtype=torch.float16, device=device),
            })
        torch.cuda.current_stream().synchronize()
    finally:
        ld.close()
    return {"config": cfg, "layers": layers, "embed_tokens": embed, "final_norm": norm,
            "lm_head": lm_head, "inv_freq": build_inv_freq(cfg.rope_theta, cfg.head_dim).to(device)}
