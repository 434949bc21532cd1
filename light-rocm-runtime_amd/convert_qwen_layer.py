#!/usr/bin/env python3
"""Hugging Face Qwen2 safetensors checkpoint -> FP32 weight bundles.

Drop-in for the reference's tools/convert_qwen_layer.py. The command line is
the same (:705-770), and so are the function names and their argument meaning,
so the reference's own tests (tests/qwen_layer_converter_test.py) run against
this module unchanged. The bundle layout is the same too:
layer_<i>/weights.json + weights.bin, then model_tail/weights.json +
weights.bin.
The two formats written are the ones qd_load_bundle reads,
lrrt.mini_decoder_weights v2 and lrrt.mini_model_tail_weights v1
(executor/qwen/weight_bundle.hpp:460-602).

Checkpoint tensors may be F32, F16 or BF16. They are widened to FP32
exactly: BF16 is the upper half of an IEEE binary32, and every binary16 value
is representable in binary32 (convert_qwen_layer.py:264-281).

A checkpoint without lm_head.weight has a tied LM head. Its tail then stores
model.embed_tokens.weight as the LM head (convert_qwen_layer.py:556-568).

Mechanism (own design; the bytes written match the reference converter's):
  * each shard is memory-mapped and only the requested tensors' bytes are
    touched. The reference reads every shard whole for every layer
    (convert_qwen_layer.py:294-296).
  * every tensor entry is validated before conversion (dtype, shape, exact
    byte length, range inside the file);
  * a tensor is streamed to the data file as soon as it is converted, and the
    manifest is written last.

For qd_load_bundle, convert every layer and the full-vocabulary tail:
  convert_qwen_layer.py --checkpoint-dir CKPT --keys 1 --all-layers \\
      --full-token-embeddings --output BUNDLE_DIR
"""

from __future__ import annotations

import argparse
import json
import mmap
import struct
import sys
from dataclasses import dataclass
from pathlib import Path
from typing import Any

import numpy as np

FORMAT = "lrrt.mini_decoder_weights"
TAIL_FORMAT = "lrrt.mini_model_tail_weights"
VERSION = 1
DECODER_VERSION = 2

# safetensors dtype -> (little-endian storage dtype, widening to float32).
# BF16 keeps the sign, exponent and top 7 mantissa bits of binary32, so the
# widening is a 16-bit left shift of the raw bits.
_WIDEN = {
    "F32": ("<f4", lambda raw: raw.astype(np.float32)),
    "F16": ("<f2", lambda raw: raw.astype(np.float32)),
    "BF16": ("<u2", lambda raw: (raw.astype(np.uint32) << 16).view(np.float32)),
}


@dataclass(frozen=True)
class DecoderLayerShape:
    """convert_qwen_layer.py:20-35."""

    keys: int
    hidden: int
    heads: int
    kv_heads: int
    head_dim: int
    intermediate: int

    @property
    def q_dim(self) -> int:
        return self.heads * self.head_dim

    @property
    def kv_dim(self) -> int:
        return self.kv_heads * self.head_dim


@dataclass(frozen=True)
class TensorMapping:
    """One bundle tensor and the checkpoint tensor it comes from (:38-42)."""

    bundle_name: str
    checkpoint_name: str
    shape: tuple[int, ...]


# ---- config -> shape -------------------------------------------------------------

def _positive_int(config: dict[str, Any], key: str) -> int:
    value = config.get(key)
    if isinstance(value, bool) or not isinstance(value, int) or value <= 0:
        raise ValueError(f"config field {key!r} must be a positive integer")
    return value


def derive_shape(config: dict[str, Any], keys: int) -> DecoderLayerShape:
    """Decoder shape from a Hugging Face config (convert_qwen_layer.py:52-93).

    head_dim defaults to hidden / heads. The kernels need an even head_dim
    (RoPE rotates pairs), heads * head_dim == hidden, and heads a multiple of
    kv_heads (grouped-query attention).
    """
    if keys <= 0:
        raise ValueError("--keys must be a positive integer")
    hidden = _positive_int(config, "hidden_size")
    heads = _positive_int(config, "num_attention_heads")
    intermediate = _positive_int(config, "intermediate_size")
    kv_heads = config.get("num_key_value_heads", heads)
    if isinstance(kv_heads, bool) or not isinstance(kv_heads, int) or kv_heads <= 0:
        raise ValueError("config field 'num_key_value_heads' must be positive")
    if heads % kv_heads != 0:
        raise ValueError(
            "the mini decoder converter expects num_attention_heads to be a "
            f"multiple of num_key_value_heads, got num_key_value_heads={kv_heads}, "
            f"num_attention_heads={heads}")
    head_dim = config.get("head_dim")
    if head_dim is None:
        if hidden % heads != 0:
            raise ValueError("hidden_size must be divisible by num_attention_heads")
        head_dim = hidden // heads
    if isinstance(head_dim, bool) or not isinstance(head_dim, int) or head_dim <= 0:
        raise ValueError("config field 'head_dim' must be a positive integer")
    if head_dim % 2:
        raise ValueError("head_dim must be even for the current RoPE kernels")
    if heads * head_dim != hidden:
        raise ValueError(
            "the current mini decoder expects heads * head_dim == hidden, "
            f"got {heads} * {head_dim} != {hidden}")
    return DecoderLayerShape(keys, hidden, heads, kv_heads, head_dim, intermediate)


def derive_rope_theta(config: dict[str, Any]) -> float:
    """rope_theta, 10000 when absent (convert_qwen_layer.py:96-100)."""
    value = config.get("rope_theta", 10000.0)
    if isinstance(value, bool) or not isinstance(value, (int, float)) or not value > 0:
        raise ValueError("config field 'rope_theta' must be a positive number")
    return float(value)


def derive_model_layer_count(config: dict[str, Any]) -> int:
    return _positive_int(config, "num_hidden_layers")


def resolve_layer_count(config: dict[str, Any], args: argparse.Namespace) -> int:
    """How many consecutive layers from args.layer to convert (:107-127)."""
    if args.layer < 0:
        raise ValueError("--layer must be non-negative")
    if args.all_layers:
        if args.layer_count != 1:
            raise ValueError("--all-layers cannot be combined with --layer-count")
        total = derive_model_layer_count(config)
        if args.layer >= total:
            raise ValueError("--layer must be smaller than config field 'num_hidden_layers'")
        return total - args.layer
    if args.layer_count <= 0:
        raise ValueError("--layer-count must be a positive integer")
    if "num_hidden_layers" in config:
        if args.layer + args.layer_count > derive_model_layer_count(config):
            raise ValueError("--layer + --layer-count exceeds config field 'num_hidden_layers'")
    return args.layer_count


# The twelve decoder tensors in bundle order (executor/qwen/weight_bundle.hpp
# reads them by name; the writer's order is the reference converter's,
# convert_qwen_layer.py:130-197). Shapes are functions of DecoderLayerShape.
_LAYER_TENSORS = (
    ("attention_norm_weight", "input_layernorm.weight", lambda s: (s.hidden,)),
    ("mlp_norm_weight", "post_attention_layernorm.weight", lambda s: (s.hidden,)),
    ("q_weight", "self_attn.q_proj.weight", lambda s: (s.q_dim, s.hidden)),
    ("k_weight", "self_attn.k_proj.weight", lambda s: (s.kv_dim, s.hidden)),
    ("v_weight", "self_attn.v_proj.weight", lambda s: (s.kv_dim, s.hidden)),
    ("q_bias", "self_attn.q_proj.bias", lambda s: (s.q_dim,)),
    ("k_bias", "self_attn.k_proj.bias", lambda s: (s.kv_dim,)),
    ("v_bias", "self_attn.v_proj.bias", lambda s: (s.kv_dim,)),
    ("out_weight", "self_attn.o_proj.weight", lambda s: (s.hidden, s.q_dim)),
    ("gate_weight", "mlp.gate_proj.weight", lambda s: (s.intermediate, s.hidden)),
    ("up_weight", "mlp.up_proj.weight", lambda s: (s.intermediate, s.hidden)),
    ("down_weight", "mlp.down_proj.weight", lambda s: (s.hidden, s.intermediate)),
)


def tensor_mappings(layer: int, shape: DecoderLayerShape) -> list[TensorMapping]:
    if layer < 0:
        raise ValueError("--layer must be non-negative")
    return [TensorMapping(name, f"model.layers.{layer}.{suffix}", dims(shape))
            for name, suffix, dims in _LAYER_TENSORS]


def tail_tensor_names() -> tuple[str, str, str]:
    return ("model.embed_tokens.weight", "model.norm.weight", "lm_head.weight")


def parse_token_ids(text: str) -> list[int]:
    """Comma-separated non-negative decimal ids (:204-220)."""
    if not text:
        raise ValueError("--token-ids must not be empty")
    ids: list[int] = []
    for item in (part.strip() for part in text.split(",")):
        if not item:
            raise ValueError("--token-ids contains an empty entry")
        try:
            value = int(item, 10)
        except ValueError as error:
            raise ValueError(f"--token-ids contains a non-integer: {item!r}") from error
        if value < 0:
            raise ValueError("--token-ids must contain non-negative integers")
        ids.append(value)
    return ids


def read_json(path: Path) -> dict[str, Any]:
    with Path(path).open("r", encoding="utf-8") as file:
        data = json.load(file)
    if not isinstance(data, dict):
        raise ValueError(f"{path} must contain a JSON object")
    return data


def _import_numpy() -> Any:
    return np


# ---- safetensors -----------------------------------------------------------------

class _Shard:
    """One memory-mapped .safetensors file.

    Layout: u64 little-endian header length N, N bytes of JSON mapping each
    tensor name to {dtype, shape, data_offsets: [begin, end)} relative to
    the byte after the header, then the tensor bytes.
    """

    def __init__(self, path: Path):
        self.path = Path(path)
        with self.path.open("rb") as file:
            head = file.read(8)
            if len(head) != 8:
                raise ValueError(f"{self.path} is not a valid safetensors file")
            (size,) = struct.unpack("<Q", head)
            body = file.read(size) if size <= (1 << 30) else b""
            if len(body) != size:
                raise ValueError(f"{self.path} has a truncated safetensors header")
            try:
                header = json.loads(body.decode("utf-8"))
            except (UnicodeDecodeError, json.JSONDecodeError) as error:
                raise ValueError(f"{self.path} has an unreadable safetensors header") from error
            if not isinstance(header, dict):
                raise ValueError(f"{self.path} safetensors header must be an object")
            self.header = header
            self.base = 8 + size
            total = self.path.stat().st_size
            self.data_len = total - self.base
            self._map = (mmap.mmap(file.fileno(), 0, access=mmap.ACCESS_READ)
                         if total > 0 else None)

    def names(self) -> set[str]:
        return {name for name in self.header if name != "__metadata__"}

    def close(self) -> None:
        if self._map is not None:
            self._map.close()
            self._map = None

    def __enter__(self) -> "_Shard":
        return self

    def __exit__(self, *exc) -> None:
        self.close()

    def tensor(self, name: str) -> np.ndarray:
        """Tensor `name` widened to a C-contiguous float32 array of its shape."""
        entry = self.header.get(name)
        if not isinstance(entry, dict):
            raise ValueError(f"{self.path} tensor {name!r} metadata is invalid")
        dtype = entry.get("dtype")
        dims = entry.get("shape")
        offsets = entry.get("data_offsets")
        if (not isinstance(dtype, str) or not isinstance(dims, list)
                or not isinstance(offsets, list) or len(offsets) != 2):
            raise ValueError(f"{self.path} tensor {name!r} metadata is incomplete")
        if dtype not in _WIDEN:
            raise ValueError(f"unsupported safetensors dtype for {name!r}: {dtype}")
        if not all(isinstance(d, int) and not isinstance(d, bool) and d >= 0 for d in dims):
            raise ValueError(f"{self.path} tensor {name!r} shape is invalid")
        if not all(isinstance(o, int) and not isinstance(o, bool) for o in offsets):
            raise ValueError(f"{self.path} tensor {name!r} data offset is invalid")
        begin, end = offsets
        if begin < 0 or end < begin or end > self.data_len:
            raise ValueError(f"{self.path} tensor {name!r} data offset is invalid")
        storage, widen = _WIDEN[dtype]
        count = 1
        for d in dims:
            count *= d
        if end - begin != count * np.dtype(storage).itemsize:
            raise ValueError(
                f"{self.path} tensor {name!r} holds {end - begin} bytes, "
                f"expected {count * np.dtype(storage).itemsize} for {dtype} {tuple(dims)}")
        if count == 0:
            return np.zeros(tuple(dims), np.float32)
        raw = np.frombuffer(self._map, dtype=storage, count=count, offset=self.base + begin)
        # widen() returns a new array, so nothing keeps the mapping alive.
        return np.ascontiguousarray(widen(raw).reshape(tuple(dims)), dtype=np.float32)


def read_safetensors(path: Path, wanted: set[str]) -> dict[str, Any]:
    """Every tensor of `wanted` that the file holds, widened to FP32 (:284-323)."""
    with _Shard(path) as shard:
        return {name: shard.tensor(name) for name in wanted if name in shard.header}


def read_safetensors_names(path: Path) -> set[str]:
    with _Shard(path) as shard:
        return shard.names()


def checkpoint_weight_map(checkpoint_dir: Path) -> dict[str, str] | None:
    """Tensor name -> shard file from *.safetensors.index.json, if present (:239-253)."""
    index_paths = sorted(Path(checkpoint_dir).glob("*.safetensors.index.json"))
    if not index_paths:
        return None
    index = read_json(index_paths[0])
    weight_map = index.get("weight_map")
    if not isinstance(weight_map, dict):
        raise ValueError(f"{index_paths[0]} is missing object field 'weight_map'")
    for name, file_name in weight_map.items():
        if not isinstance(name, str) or not isinstance(file_name, str):
            raise ValueError(f"{index_paths[0]} contains invalid weight_map entries")
    return dict(weight_map)


def _safetensor_files(checkpoint_dir: Path) -> list[Path]:
    files = sorted(Path(checkpoint_dir).glob("*.safetensors"))
    if not files:
        raise FileNotFoundError(f"no .safetensors files found in {checkpoint_dir}")
    return files


def _shard_path(checkpoint_dir: Path, file_name: str) -> Path:
    # An index may only name files inside the checkpoint directory.
    part = Path(file_name)
    if part.is_absolute() or len(part.parts) != 1 or part.name in ("", ".", ".."):
        raise ValueError(f"checkpoint index names a shard outside the directory: {file_name!r}")
    return Path(checkpoint_dir) / part


def checkpoint_tensor_names(checkpoint_dir: Path) -> set[str]:
    weight_map = checkpoint_weight_map(checkpoint_dir)
    if weight_map is not None:
        return set(weight_map)
    names: set[str] = set()
    for path in _safetensor_files(checkpoint_dir):
        names |= read_safetensors_names(path)
    return names


def load_tensors(checkpoint_dir: Path, mappings: list[TensorMapping]) -> dict[str, Any]:
    """The mappings' checkpoint tensors as FP32 arrays (:343-369).

    With an index, only the shards that hold a wanted tensor are opened;
    without one, shards are scanned in name order until all are found.
    Raises KeyError naming every missing tensor.
    """
    wanted = {m.checkpoint_name for m in mappings}
    weight_map = checkpoint_weight_map(checkpoint_dir)
    tensors: dict[str, Any] = {}
    if weight_map is not None:
        missing = sorted(wanted - set(weight_map))
        if missing:
            raise KeyError("checkpoint index is missing tensors: " + ", ".join(missing))
        by_shard: dict[str, set[str]] = {}
        for name in wanted:
            by_shard.setdefault(weight_map[name], set()).add(name)
        for file_name in sorted(by_shard):
            tensors.update(read_safetensors(_shard_path(checkpoint_dir, file_name),
                                            by_shard[file_name]))
    else:
        for path in _safetensor_files(checkpoint_dir):
            tensors.update(read_safetensors(path, wanted - set(tensors)))
            if len(tensors) == len(wanted):
                break
    missing = sorted(wanted - set(tensors))
    if missing:
        raise KeyError("checkpoint is missing tensors: " + ", ".join(missing))
    return tensors


def validate_no_unsupported_attention_biases(
        checkpoint_dir: Path, layer: int, available_names: set[str] | None = None) -> None:
    """Qwen2 has q/k/v biases but no o_proj bias; the bundle has no slot for one (:372-385)."""
    if available_names is None:
        available_names = checkpoint_tensor_names(checkpoint_dir)
    name = f"model.layers.{layer}.self_attn.o_proj.bias"
    if name in available_names:
        raise ValueError("output projection biases are not supported by the mini decoder "
                         "converter: " + name)


def convert_tensor(value: Any, expected_shape: tuple[int, ...], name: str) -> Any:
    array = np.ascontiguousarray(value, dtype=np.float32)
    if tuple(array.shape) != tuple(expected_shape):
        raise ValueError(
            f"tensor {name!r} has shape {tuple(array.shape)}, expected {tuple(expected_shape)}")
    return array


# ---- bundle writers --------------------------------------------------------------

def _validate_data_file_name(data_file_name: str) -> None:
    """The data file sits beside its manifest: one relative component, no '..'."""
    part = Path(data_file_name)
    if (not data_file_name or part.is_absolute() or ".." in part.parts
            or len(part.parts) != 1):
        raise ValueError("--data-file must be a single relative file name")


def _write_tensors(output_manifest: Path, data_file_name: str,
                   named: list[tuple[str, np.ndarray]]) -> list[dict[str, int | str]]:
    """Streams FP32 tensors back to back; returns the manifest's tensor entries."""
    entries: list[dict[str, int | str]] = []
    offset = 0
    with (output_manifest.parent / data_file_name).open("wb") as data:
        for name, array in named:
            flat = np.ascontiguousarray(array, dtype="<f4").reshape(-1)
            data.write(memoryview(flat).cast("B"))
            entries.append({"name": name, "offset": offset, "count": int(flat.size)})
            offset += flat.size * 4
    return entries


def _write_manifest(output_manifest: Path, manifest: dict[str, Any]) -> None:
    with output_manifest.open("w", encoding="utf-8") as file:
        json.dump(manifest, file, indent=2)
        file.write("\n")


def write_bundle(output_manifest: Path, data_file_name: str, shape: DecoderLayerShape,
                 tensors: dict[str, Any], rope_theta: float = 10000.0) -> None:
    """One decoder layer as lrrt.mini_decoder_weights v2 (:399-458)."""
    _validate_data_file_name(data_file_name)
    output_manifest = Path(output_manifest)
    named: list[tuple[str, np.ndarray]] = []
    for mapping in tensor_mappings(0, shape):
        name = mapping.bundle_name
        if name not in tensors:
            raise KeyError(f"missing converted tensor: {name}")
        array = np.asarray(tensors[name], dtype=np.float32)
        expected = int(np.prod(mapping.shape))
        if array.size != expected:
            raise ValueError(f"tensor {name!r} has {array.size} values, expected {expected}")
        named.append((name, array))
    output_manifest.parent.mkdir(parents=True, exist_ok=True)
    entries = _write_tensors(output_manifest, data_file_name, named)
    _write_manifest(output_manifest, {
        "format": FORMAT,
        "version": DECODER_VERSION,
        "dtype": "f32",
        "data": data_file_name,
        "keys": shape.keys,
        "hidden": shape.hidden,
        "heads": shape.heads,
        "kv_heads": shape.kv_heads,
        "head_dim": shape.head_dim,
        "intermediate": shape.intermediate,
        "rope_theta": rope_theta,
        "tensors": entries,
    })


def _write_tail_bundle(output_manifest: Path, data_file_name: str, hidden: int,
                       token_ids: list[int], token_embeddings: Any, final_norm_weight: Any,
                       lm_head_weight: Any) -> None:
    """Embedding rows of token_ids, final norm and LM head as
    lrrt.mini_model_tail_weights v1 (:461-529)."""
    _validate_data_file_name(data_file_name)
    if not token_ids:
        raise ValueError("at least one token id is required")
    token_embeddings = np.asarray(token_embeddings, dtype=np.float32)
    final_norm_weight = np.asarray(final_norm_weight, dtype=np.float32)
    lm_head_weight = np.asarray(lm_head_weight, dtype=np.float32)
    if token_embeddings.shape != (len(token_ids), hidden):
        raise ValueError(f"token embeddings have shape {token_embeddings.shape}, "
                         f"expected {(len(token_ids), hidden)}")
    if final_norm_weight.shape != (hidden,):
        raise ValueError(f"model.norm.weight has shape {final_norm_weight.shape}, "
                         f"expected {(hidden,)}")
    if lm_head_weight.ndim != 2 or lm_head_weight.shape[1] != hidden:
        raise ValueError("lm_head.weight must have shape [vocab, hidden], got "
                         f"{lm_head_weight.shape}")
    vocab = int(lm_head_weight.shape[0])
    for token_id in token_ids:
        if not 0 <= token_id < vocab:
            raise ValueError(f"token id must be in [0, {vocab}), got {token_id}")
    output_manifest = Path(output_manifest)
    output_manifest.parent.mkdir(parents=True, exist_ok=True)
    entries = _write_tensors(output_manifest, data_file_name, [
        ("token_embeddings", token_embeddings),
        ("final_norm_weight", final_norm_weight),
        ("lm_head_weight", lm_head_weight),
    ])
    _write_manifest(output_manifest, {
        "format": TAIL_FORMAT,
        "version": VERSION,
        "dtype": "f32",
        "data": data_file_name,
        "hidden": hidden,
        "vocab": vocab,
        "token_ids": [int(t) for t in token_ids],
        "tensors": entries,
    })


# ---- conversion ------------------------------------------------------------------

def _convert_tail(checkpoint_dir: Path, output: Path, data_file: str, hidden: int,
                  token_ids: list[int], full_token_embeddings: bool) -> None:
    """The model tail; a checkpoint without lm_head.weight has a tied head (:532-593)."""
    embed_name, norm_name, head_name = tail_tensor_names()
    base = [TensorMapping("embed_tokens", embed_name, (1,)),
            TensorMapping("final_norm_weight", norm_name, (hidden,))]
    try:
        tensors = load_tensors(checkpoint_dir,
                               base + [TensorMapping("lm_head_weight", head_name, (1, hidden))])
    except KeyError:
        tensors = load_tensors(checkpoint_dir, base)
        tensors[head_name] = tensors[embed_name]
    embed = tensors[embed_name]
    if embed.ndim != 2 or embed.shape[1] != hidden:
        raise ValueError(f"model.embed_tokens.weight must have shape [vocab, hidden], got "
                         f"{embed.shape}")
    if full_token_embeddings:
        token_ids = list(range(int(embed.shape[0])))
        rows = embed
    else:
        for token_id in token_ids:
            if not 0 <= token_id < embed.shape[0]:
                raise ValueError(f"token id must be in [0, {embed.shape[0]}), got {token_id}")
        rows = embed[token_ids]
    _write_tail_bundle(output, data_file, hidden, token_ids, rows, tensors[norm_name],
                       tensors[head_name])


def _convert_layer(checkpoint_dir: Path, shape: DecoderLayerShape, rope_theta: float,
                   layer: int, output: Path, data_file: str,
                   available_names: set[str] | None) -> None:
    """One decoder layer (:596-632). Absent q/k/v biases are written as zeros."""
    mappings = tensor_mappings(layer, shape)
    if available_names is None:
        available_names = checkpoint_tensor_names(checkpoint_dir)
    validate_no_unsupported_attention_biases(checkpoint_dir, layer, available_names)
    present = [m for m in mappings
               if not m.bundle_name.endswith("_bias") or m.checkpoint_name in available_names]
    loaded = load_tensors(checkpoint_dir, present)
    converted = {
        m.bundle_name: (convert_tensor(loaded[m.checkpoint_name], m.shape, m.checkpoint_name)
                        if m.checkpoint_name in loaded else np.zeros(m.shape, np.float32))
        for m in mappings
    }
    write_bundle(output, data_file, shape, converted, rope_theta)


def convert_checkpoint(args: argparse.Namespace) -> None:
    """The command (:635-699): one layer bundle, a directory of layers + tail,
    or the tail alone."""
    checkpoint_dir = Path(args.checkpoint_dir).resolve()
    config = read_json(Path(args.config).resolve() if args.config
                       else checkpoint_dir / "config.json")
    shape = derive_shape(config, args.keys)
    rope_theta = derive_rope_theta(config)
    weight_map = checkpoint_weight_map(checkpoint_dir)
    available_names = set(weight_map) if weight_map is not None else None
    layer_count = resolve_layer_count(config, args)
    token_ids = parse_token_ids(args.token_ids)
    output = Path(args.output)
    as_directory = args.all_layers or args.bundle_directory or layer_count > 1

    def tail() -> None:
        manifest = output / "model_tail" / "weights.json"
        _convert_tail(checkpoint_dir, manifest, args.data_file, shape.hidden, token_ids,
                      args.full_token_embeddings)
        print(f"wrote Qwen mini model tail: {manifest}")

    if args.tail_only:
        if output.suffix:
            raise ValueError("--output must be a directory when writing model tail")
        tail()
    elif not as_directory:
        _convert_layer(checkpoint_dir, shape, rope_theta, args.layer, output, args.data_file,
                       available_names)
        print(f"wrote Qwen mini decoder weight bundle: {output}")
    else:
        if output.suffix:
            raise ValueError("--output must be a directory when writing multiple decoder layers")
        for layer in range(args.layer, args.layer + layer_count):
            manifest = output / f"layer_{layer}" / "weights.json"
            _convert_layer(checkpoint_dir, shape, rope_theta, layer, manifest, args.data_file,
                           available_names)
            print(f"wrote Qwen mini decoder layer {layer}: {manifest}")
        tail()


def parse_args(argv: list[str]) -> argparse.Namespace:
    """Same flags as convert_qwen_layer.py:705-770."""
    p = argparse.ArgumentParser(
        description="Convert local Hugging Face Qwen decoder layers into FP32 mini decoder "
                    "weight bundles.")
    p.add_argument("--checkpoint-dir", required=True, type=Path)
    p.add_argument("--config", type=Path, help="defaults to CHECKPOINT_DIR/config.json")
    p.add_argument("--layer", default=0, type=int)
    p.add_argument("--layer-count", default=1, type=int,
                   help="consecutive layers to convert; above 1, --output is a directory "
                        "holding layer_<index>/weights.json")
    p.add_argument("--all-layers", action="store_true",
                   help="convert --layer through num_hidden_layers - 1 into a directory")
    p.add_argument("--tail-only", action="store_true",
                   help="write only model_tail/weights.json under --output")
    p.add_argument("--bundle-directory", action="store_true",
                   help="write a directory bundle (layer_<index> + model_tail) even for "
                        "one layer")
    p.add_argument("--keys", required=True, type=int)
    p.add_argument("--token-ids", default="0",
                   help="comma-separated token ids whose embedding rows the tail stores")
    p.add_argument("--full-token-embeddings", action="store_true",
                   help="store every embedding row in vocabulary order (needed to feed "
                        "generated tokens back, and by qd_load_bundle)")
    p.add_argument("--output", required=True, type=Path)
    p.add_argument("--data-file", default="weights.bin")
    return p.parse_args(argv)


def main(argv: list[str]) -> int:
    try:
        convert_checkpoint(parse_args(argv))
        return 0
    except Exception as error:  # the command's contract: one line on stderr, status 1
        print(f"convert_qwen_layer.py: {error}", file=sys.stderr)
        return 1


if __name__ == "__main__":
    raise SystemExit(main(sys.argv[1:]))
