"""A converted checkpoint decodes on the GPU exactly as the oracle does.

Chain under test: BF16 safetensors shards with an index and a tied head
-> convert_qwen_layer.py -> qd_load_bundle -> prefill and decode through the
C ABI. The oracle gets the same weights straight from the checkpoint values
(widened by torch, not by the converter). Bars: weights on the device
bit-exact with the checkpoint; logits max|gpu - ref| / max|ref| <= 1e-4;
greedy tokens identical where the oracle's top-1/top-2 margin > 1e-3.
"""
import numpy as np
import pytest

import convert_qwen_layer as cq
import qwen_decode as qd
import qwen_oracle as qo
from ckpt_util import qwen_checkpoint

pytestmark = pytest.mark.gpu

LOGIT_RTOL = 1e-4
MARGIN = 1e-3
LAYERS, VOCAB, THETA = 2, 1024, 10000.0

HF = ["input_layernorm.weight", "post_attention_layernorm.weight", "self_attn.q_proj.weight",
      "self_attn.k_proj.weight", "self_attn.v_proj.weight", "self_attn.q_proj.bias",
      "self_attn.k_proj.bias", "self_attn.v_proj.bias", "self_attn.o_proj.weight",
      "mlp.gate_proj.weight", "mlp.up_proj.weight", "mlp.down_proj.weight"]  # oracle kinds 0..11


def say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def rel_err(a, b):
    return float(np.abs(a.astype(np.float64) - b).max() / max(np.abs(b).max(), 1e-30))


def test_converted_bf16_checkpoint_decodes_like_oracle(tmp_path):
    say(f"converter: BF16 checkpoint, {LAYERS} layers, vocab {VOCAB}, rope_theta {THETA}")
    values = qwen_checkpoint(tmp_path / "ckpt", hidden=896, heads=14, kv_heads=2, intermediate=4864,
                             vocab=VOCAB, layers=LAYERS, dtype="BF16", tied=True, shards=2, seed=11,
                             rope_theta=THETA, weight_std=0.02)
    out = tmp_path / "bundle"
    assert cq.main(["--checkpoint-dir", str(tmp_path / "ckpt"), "--keys", "1", "--all-layers",
                    "--full-token-embeddings", "--output", str(out)]) == 0

    shape = qo.ModelShape(layers=LAYERS, vocab=VOCAB, rope_theta=THETA)
    model = qo.Model(shape)
    for layer in range(LAYERS):
        for kind, suffix in enumerate(HF):
            model.tensor(layer, kind)[:] = values[f"model.layers.{layer}.{suffix}"].reshape(-1)
    model.tensor(0, 0x100)[:] = values["model.embed_tokens.weight"].reshape(-1)
    model.tensor(0, 0x101)[:] = values["model.norm.weight"]

    say("converter: load bundle into the engine")
    eng = qd.Engine(layers=LAYERS, vocab=VOCAB, capacity=64, max_batch=1)
    try:
        eng.load_bundle(str(out))
        for layer in range(LAYERS):
            for kind, suffix in enumerate(HF):
                want = values[f"model.layers.{layer}.{suffix}"].reshape(-1)
                got = eng.read_weight(layer, kind, want.size)
                assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (layer, suffix)
        embed = values["model.embed_tokens.weight"].reshape(-1)
        assert np.array_equal(eng.read_weight(0, 0x100, embed.size), embed)
        assert np.array_equal(eng.read_weight(0, 0x102, embed.size), embed)

        prompt = qo.fill_tokens(6, 3, 0x300000, VOCAB)
        say(f"converter: prefill {prompt.tolist()} + 6 greedy steps")
        cache = qo.Cache(model, 64)
        eng.kv_reset(0, 0)
        tok, _, logits = eng.prefill(0, prompt)
        rtok, _, rlogits = cache.prefill(prompt)
        errs = []
        for i in range(7):
            err = rel_err(logits, rlogits)
            errs.append(err)
            assert err <= LOGIT_RTOL, f"step {i}: logits rel err {err:.3e}"
            assert tok == int(np.argmax(logits))
            top2 = np.partition(rlogits, -2)[-2:]
            if top2[1] - top2[0] > MARGIN:
                assert tok == rtok, f"step {i}: token {tok} != oracle {rtok}"
            if i == 6:
                break
            feed = rtok
            tok, _, logits = eng.step(0, feed)
            rtok, _, rlogits = cache.decode_step(feed, len(prompt) + i)
        say(f"converter: max logits rel err {max(errs):.3e}")
        cache.close()
    finally:
        eng.close()
        model.close()
