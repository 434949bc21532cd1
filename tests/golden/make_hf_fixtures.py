"""Writes the Hugging Face Qwen2 golden fixtures under tests/golden/.

The reference's CPU validation path is Hugging Face `AutoModelForCausalLM`
in FP32 eager mode, run step by step over the full prefix without a KV cache
(tools/run_qwen_e2e.py:369-400). Its arithmetic lives in the third-party
`transformers` package (unpinned by the reference; this container has 5.15.0
with torch 2.10.0), not in /root/reference. This script restates that call
offline: `Qwen2ForCausalLM(Qwen2Config(...))` with weights from the oracle's
seeded generator, then greedy decoding with a full-prefix forward at every
step. It stores only seeds, shapes, tokens, logits and RoPE tables, so the
oracle tests regenerate the weights and compare.

Run in this container only:  python tests/golden/make_hf_fixtures.py
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))

import qwen_oracle as qo  # noqa: E402

PROMPT_STREAM = 0x300000

CASES = {
    # Tiny two-layer model: every composition rule at a size HF runs instantly.
    "hf_tiny": dict(shape=qo.ModelShape(hidden=256, heads=4, kv_heads=2, head_dim=64,
                                        intermediate=512, vocab=512, layers=2),
                    seed=11, prompt=7, steps=6),
    # One real-shape Qwen2.5-0.5B layer with a short vocabulary.
    "hf_qwen_layer": dict(shape=qo.ModelShape(layers=1, vocab=1024), seed=12, prompt=5, steps=4),
}

ROPE_POSITIONS = np.array([0, 1, 2, 3, 127, 128, 511, 576, 2047, 4095, 4127], np.int64)


def build_hf(model: qo.Model):
    import torch
    from transformers import Qwen2Config, Qwen2ForCausalLM

    s = model.shape
    cfg = Qwen2Config(
        vocab_size=s.vocab, hidden_size=s.hidden, intermediate_size=s.intermediate,
        num_hidden_layers=s.layers, num_attention_heads=s.heads,
        num_key_value_heads=s.kv_heads, head_dim=s.head_dim, hidden_act="silu",
        max_position_embeddings=8192, rms_norm_eps=s.eps, rope_theta=s.rope_theta,
        tie_word_embeddings=True, use_sliding_window=False, attention_dropout=0.0,
    )
    cfg._attn_implementation = "eager"
    hf = Qwen2ForCausalLM(cfg).to(torch.float32).eval()

    def t(layer, kind, shape):
        return torch.from_numpy(model.tensor(layer, kind).reshape(shape).copy())

    H, Q, KV, I = s.hidden, s.heads * s.head_dim, s.kv_heads * s.head_dim, s.intermediate
    sd = {"model.embed_tokens.weight": t(0, qo.EMBED, (s.vocab, H)),
          "model.norm.weight": t(0, qo.FINAL_NORM, (H,)),
          "lm_head.weight": t(0, qo.EMBED, (s.vocab, H))}
    for i in range(s.layers):
        p = f"model.layers.{i}."
        sd[p + "input_layernorm.weight"] = t(i, qo.ATTN_NORM, (H,))
        sd[p + "post_attention_layernorm.weight"] = t(i, qo.MLP_NORM, (H,))
        sd[p + "self_attn.q_proj.weight"] = t(i, qo.Q_W, (Q, H))
        sd[p + "self_attn.q_proj.bias"] = t(i, qo.Q_B, (Q,))
        sd[p + "self_attn.k_proj.weight"] = t(i, qo.K_W, (KV, H))
        sd[p + "self_attn.k_proj.bias"] = t(i, qo.K_B, (KV,))
        sd[p + "self_attn.v_proj.weight"] = t(i, qo.V_W, (KV, H))
        sd[p + "self_attn.v_proj.bias"] = t(i, qo.V_B, (KV,))
        sd[p + "self_attn.o_proj.weight"] = t(i, qo.O_W, (H, Q))
        sd[p + "mlp.gate_proj.weight"] = t(i, qo.GATE_W, (I, H))
        sd[p + "mlp.up_proj.weight"] = t(i, qo.UP_W, (I, H))
        sd[p + "mlp.down_proj.weight"] = t(i, qo.DOWN_W, (H, I))
    missing, unexpected = hf.load_state_dict(sd, strict=False)
    missing = [m for m in missing if "rotary" not in m]
    if missing or unexpected:
        raise RuntimeError(f"state dict mismatch: missing={missing} unexpected={unexpected}")
    hf.tie_weights()
    return hf


def make_case(name: str, shape: qo.ModelShape, seed: int, prompt: int, steps: int):
    import torch

    model = qo.Model(shape, tied=True)
    model.fill_synthetic(seed)
    hf = build_hf(model)
    prompt_ids = qo.fill_tokens(prompt, seed, PROMPT_STREAM, shape.vocab)
    ids = [int(x) for x in prompt_ids]
    logits_all, tokens = [], []
    with torch.inference_mode():
        for _ in range(steps):
            out = hf(input_ids=torch.tensor([ids], dtype=torch.long)).logits[0, -1].float()
            logits_all.append(out.numpy().astype(np.float32))
            tok = int(torch.argmax(out).item())
            tokens.append(tok)
            ids.append(tok)
        pos = torch.tensor([ROPE_POSITIONS.tolist()], dtype=torch.long)
        dummy = torch.zeros((1, len(ROPE_POSITIONS), shape.hidden), dtype=torch.float32)
        cos, sin = hf.model.rotary_emb(dummy, pos)
    np.savez(
        os.path.join(HERE, f"{name}.npz"),
        shape=np.array([shape.hidden, shape.heads, shape.kv_heads, shape.head_dim,
                        shape.intermediate, shape.vocab, shape.layers], np.int64),
        eps=np.float32(shape.eps), rope_theta=np.float32(shape.rope_theta),
        seed=np.int64(seed), prompt=prompt_ids.astype(np.int64),
        tokens=np.array(tokens, np.int64), logits=np.stack(logits_all),
        rope_positions=ROPE_POSITIONS, rope_cos=cos[0].numpy().astype(np.float32),
        rope_sin=sin[0].numpy().astype(np.float32),
    )
    print(f"{name}: prompt={prompt_ids.tolist()} tokens={tokens}")


def main():
    for name, case in CASES.items():
        make_case(name, **case)


if __name__ == "__main__":
    main()
