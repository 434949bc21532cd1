"""Synthetic Hugging Face-style Qwen2 checkpoints for the converter tests.

The safetensors files are written here with a writer independent of the
converter's reader: an 8-byte little-endian header length, then a JSON header
padded with spaces to a multiple of 8, then the tensor bytes. BF16 values
come from torch's own float32 -> bfloat16 rounding and widening, so the
expected FP32 values do not share code with the converter.
"""
from __future__ import annotations

import json
import struct
from pathlib import Path

import numpy as np
import torch


def bf16_round(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """(raw bfloat16 bits as uint16, their float32 values), both from torch."""
    t = torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.bfloat16)
    bits = t.view(torch.int16).numpy().view(np.uint16).copy()
    return bits, t.to(torch.float32).numpy().copy()


def encode(values: np.ndarray, dtype: str) -> tuple[np.ndarray, np.ndarray]:
    """(stored array for safetensors `dtype`, the float32 values it holds)."""
    if dtype == "BF16":
        return bf16_round(values)
    if dtype == "F16":
        h = np.ascontiguousarray(values, np.float16)
        return h, torch.from_numpy(h).to(torch.float32).numpy()
    f = np.ascontiguousarray(values, np.float32)
    return f, f.copy()


def write_safetensors(path: Path, tensors: dict[str, tuple[str, np.ndarray]],
                      metadata: dict[str, str] | None = None) -> None:
    header: dict = {}
    blobs, off = [], 0
    for name, (dtype, arr) in tensors.items():
        blob = np.ascontiguousarray(arr).tobytes()
        header[name] = {"dtype": dtype, "shape": list(arr.shape), "data_offsets": [off, off + len(blob)]}
        blobs.append(blob)
        off += len(blob)
    if metadata is not None:
        header["__metadata__"] = metadata
    text = json.dumps(header).encode()
    text += b" " * (-len(text) % 8)
    Path(path).write_bytes(struct.pack("<Q", len(text)) + text + b"".join(blobs))


def layer_shapes(hidden, heads, kv_heads, intermediate):
    hd = hidden // heads
    q, kv = heads * hd, kv_heads * hd
    return {
        "input_layernorm.weight": (hidden,),
        "post_attention_layernorm.weight": (hidden,),
        "self_attn.q_proj.weight": (q, hidden),
        "self_attn.k_proj.weight": (kv, hidden),
        "self_attn.v_proj.weight": (kv, hidden),
        "self_attn.q_proj.bias": (q,),
        "self_attn.k_proj.bias": (kv,),
        "self_attn.v_proj.bias": (kv,),
        "self_attn.o_proj.weight": (hidden, q),
        "mlp.gate_proj.weight": (intermediate, hidden),
        "mlp.up_proj.weight": (intermediate, hidden),
        "mlp.down_proj.weight": (hidden, intermediate),
    }


def qwen_checkpoint(directory: Path, *, hidden=8, heads=2, kv_heads=1, intermediate=12, vocab=10,
                    layers=3, dtype="BF16", tied=True, shards=2, seed=0, rope_theta=1e6,
                    biases=True, weight_std=0.5) -> dict[str, np.ndarray]:
    """Writes config.json and the shards (plus an index when shards > 1).

    Returns checkpoint tensor name -> the float32 values stored. Layer l's
    tensors go to shard l % shards; the tail tensors go to the last shard.
    """
    directory = Path(directory)
    directory.mkdir(parents=True, exist_ok=True)
    rng = np.random.default_rng(seed)
    values: dict[str, np.ndarray] = {}
    stored: list[dict[str, tuple[str, np.ndarray]]] = [{} for _ in range(shards)]

    def add(name, shard, raw):
        arr, val = encode(raw, dtype)
        stored[shard][name] = (dtype, arr)
        values[name] = val

    for layer in range(layers):
        for suffix, shape in layer_shapes(hidden, heads, kv_heads, intermediate).items():
            if suffix.endswith(".bias") and not biases:
                continue
            if "layernorm" in suffix:
                raw = 1.0 + 0.1 * rng.standard_normal(shape)
            elif suffix.endswith(".bias"):
                raw = 0.2 * rng.standard_normal(shape)
            else:
                raw = weight_std * rng.standard_normal(shape)
            add(f"model.layers.{layer}.{suffix}", layer % shards, raw)
    add("model.embed_tokens.weight", shards - 1, weight_std * rng.standard_normal((vocab, hidden)))
    add("model.norm.weight", shards - 1, 1.0 + 0.1 * rng.standard_normal(hidden))
    if not tied:
        add("lm_head.weight", shards - 1, weight_std * rng.standard_normal((vocab, hidden)))

    if shards == 1:
        write_safetensors(directory / "model.safetensors", stored[0], {"format": "pt"})
    else:
        weight_map = {}
        for i, part in enumerate(stored):
            fname = f"model-{i + 1:05d}-of-{shards:05d}.safetensors"
            write_safetensors(directory / fname, part, {"format": "pt"})
            weight_map.update({name: fname for name in part})
        (directory / "model.safetensors.index.json").write_text(
            json.dumps({"metadata": {"total_size": 0}, "weight_map": weight_map}))
    config = {
        "architectures": ["Qwen2ForCausalLM"],
        "hidden_size": hidden,
        "num_attention_heads": heads,
        "num_key_value_heads": kv_heads,
        "intermediate_size": intermediate,
        "num_hidden_layers": layers,
        "vocab_size": vocab,
        "rope_theta": rope_theta,
        "rms_norm_eps": 1e-6,
        "tie_word_embeddings": tied,
    }
    (directory / "config.json").write_text(json.dumps(config))
    return values
