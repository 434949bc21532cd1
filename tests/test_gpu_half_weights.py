"""GPU tests of BF16 and FP16 decoder weights with an FP32 tail (the
reference's reduced-precision modes, examples/qwen/README.md:291-300).

Such an engine stores the decoder layers' matrices (wqkv, wo, gate, up, down)
as BF16 or IEEE FP16, rounded to nearest even from the FP32 values it is
given, and keeps biases, norms, embeddings and the LM head in FP32. Its
kernels (the stream-ordered ones and the resident megakernel) widen each
weight exactly and compute in FP32, in the order the FP32 kernels use. So,
for each storage type:

* its weights read back as the FP32 engine's weights rounded to BF16 / FP16,
  bit for bit (numpy rounding, written here independently of the engine);
* its decode equals, bit for bit, an FP32 engine loaded with those rounded
  weights: logits, greedy tokens and K/V rows, through the step loop and
  through generation (both engines on their resident kernels);
* at full model size its resident generation equals its own stream-ordered
  kernels bit for bit (tokens, logits, K/V rows) at config 2's context;
* it matches the oracle computing with the same rounded weights, at the
  logits bar of the FP32 path (max|delta| / max|ref| <= 1e-4).
"""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.join(os.path.dirname(__file__), "..")
sys.path.insert(0, os.path.join(ROOT, "light-rocm-runtime_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

import qwen_decode as qd  # noqa: E402
import qwen_oracle as qo  # noqa: E402

pytestmark = pytest.mark.gpu

LAYERS, VOCAB = 2, 1024
LOGIT_RTOL = 1e-4
MARGIN = 1e-3
MATRICES = (qo.Q_W, qo.K_W, qo.V_W, qo.O_W, qo.GATE_W, qo.UP_W, qo.DOWN_W)
SIZES = [896, 896, 896 * 896, 128 * 896, 128 * 896, 896, 128, 128, 896 * 896, 4864 * 896, 4864 * 896,
         896 * 4864]
PROMPT_STREAM = 0x310000


def say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """FP32 values rounded to the nearest BF16 (ties to even), as FP32."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32)


def f16_round(x: np.ndarray) -> np.ndarray:
    """FP32 values rounded to the nearest IEEE half (ties to even), as FP32."""
    return np.ascontiguousarray(x, np.float32).astype(np.float16).astype(np.float32)


ROUND = {"bf16": bf16_round, "f16": f16_round}
DTYPES = pytest.mark.parametrize("dtype", ["bf16", "f16"])


def rel_err(a, b):
    return float(np.abs(a.astype(np.float64) - b).max() / max(np.abs(b).max(), 1e-30))


def margin(logits):
    top2 = np.partition(logits, -2)[-2:]
    return float(top2[1] - top2[0])


def engine(dtype, capacity=64):
    return qd.Engine(layers=LAYERS, vocab=VOCAB, capacity=capacity, max_batch=1, decoder_dtype=dtype)


def write_bundle(eng, directory):
    """The engine's weights (as it reads them back) as a reference bundle."""
    for layer in range(LAYERS):
        d = os.path.join(directory, f"layer_{layer}")
        os.makedirs(d)
        tensors = np.concatenate([eng.read_weight(layer, k, n) for k, n in enumerate(SIZES)])
        qd.bundle_write_layer(os.path.join(d, "weights.json"), "weights.bin", [64, 896, 14, 2, 64, 4864],
                              1e6, tensors)
    d = os.path.join(directory, "model_tail")
    os.makedirs(d)
    emb = eng.read_weight(0, qd.EMBED, VOCAB * 896)
    qd.bundle_write_tail(os.path.join(d, "weights.json"), "weights.bin", 896, VOCAB, np.arange(VOCAB), emb,
                         eng.read_weight(0, qd.FINAL_NORM, 896), emb)


@DTYPES
def test_half_weights_are_the_rounded_fp32_weights(dtype):
    say(f"{dtype} engine: weights = FP32 synthetic weights rounded to {dtype}")
    e32, e16 = engine("f32"), engine(dtype)
    try:
        e32.load_synthetic(1)
        e16.load_synthetic(1)
        for layer in range(LAYERS):
            for kind, n in enumerate(SIZES):
                w32 = e32.read_weight(layer, kind, n)
                w16 = e16.read_weight(layer, kind, n)
                want = ROUND[dtype](w32) if kind in MATRICES else w32
                assert np.array_equal(w16.view(np.uint32), want.view(np.uint32)), (layer, kind)
                if kind in MATRICES:
                    assert not np.array_equal(w16, w32), (layer, kind)  # really rounded
        assert np.array_equal(e16.read_weight(0, qd.EMBED, VOCAB * 896), e32.read_weight(0, qd.EMBED, VOCAB * 896))
        # Half the matrix bytes on the device, and the resident kernel on.
        saved = LAYERS * 2 * (896 * 1152 + 896 * 896 + 3 * 4864 * 896)
        assert e32.device_bytes() - e16.device_bytes() >= saved * 0.99
        assert e16.resident_grid() == e32.resident_grid() > 0
    finally:
        e32.close()
        e16.close()


@DTYPES
def test_half_decode_equals_fp32_engine_on_the_rounded_weights(dtype, tmp_path):
    say(f"{dtype} engine vs FP32 engine loaded with the rounded weights: step loop + generate")
    e16, e32 = engine(dtype), engine("f32")
    try:
        e16.load_synthetic(1)
        write_bundle(e16, str(tmp_path))
        e32.load_bundle(str(tmp_path))
        assert e32.resident_grid() > 0 and e16.resident_grid() > 0
        prompt = qo.fill_tokens(5, 1, PROMPT_STREAM, VOCAB).tolist()
        feeds = {}
        for name, eng in (("half", e16), ("f32", e32)):
            eng.kv_reset(0, 0)
            out = [eng.step(0, t) for t in prompt]
            feeds[name] = out
        for (t16, _, l16), (t32, _, l32) in zip(feeds["half"], feeds["f32"]):
            assert t16 == t32 and np.array_equal(l16, l32)
        first = feeds["half"][-1][0]
        g16 = e16.generate(0, first, 6, want_logits=True)
        g32 = e32.generate(0, first, 6, want_logits=True)
        assert g16[0].tolist() == g32[0].tolist()
        assert np.array_equal(g16[2], g32[2])
        for layer in range(LAYERS):
            k16, v16 = e16.read_kv(0, layer, 0, len(prompt) + 6)
            k32, v32 = e32.read_kv(0, layer, 0, len(prompt) + 6)
            assert np.array_equal(k16, k32) and np.array_equal(v16, v32), layer
    finally:
        e16.close()
        e32.close()


@DTYPES
def test_half_decode_matches_oracle_on_the_rounded_weights(dtype):
    say(f"{dtype} engine vs oracle computing with {dtype}-rounded matrices")
    model = qo.Model(qo.ModelShape(layers=LAYERS, vocab=VOCAB))
    model.fill_synthetic(1)
    for layer in range(LAYERS):
        for kind in MATRICES:
            t = model.tensor(layer, kind)
            t[:] = ROUND[dtype](t)
    eng = engine(dtype)
    try:
        eng.load_synthetic(1)
        prompt = qo.fill_tokens(7, 1, PROMPT_STREAM + 1, VOCAB).tolist()
        eng.kv_reset(0, 0)
        first, _, logits = eng.prefill(0, prompt)
        cache = qo.Cache(model, 64)
        rtok, _, rlog = cache.prefill(prompt)
        assert rel_err(logits, rlog) <= LOGIT_RTOL
        assert first == rtok or margin(rlog) <= MARGIN
        toks, _, glog = eng.generate(0, first, 5, want_logits=True)
        feed = first
        for i, t in enumerate(toks.tolist()):
            rtok, _, rlog = cache.decode_step(feed, len(prompt) + i)
            err = rel_err(glog[i], rlog)
            assert err <= LOGIT_RTOL, f"step {i}: logits rel err {err:.3e}"
            assert t == int(np.argmax(glog[i]))
            if margin(rlog) > MARGIN:
                assert t == rtok, f"step {i}: token {t} != oracle {rtok}"
            feed = t
        gk, _ = eng.read_kv(0, 1, len(prompt) + 4, 1)
        assert rel_err(gk[0], cache.layer(1, False)[len(prompt) + 4]) <= 1e-4
        cache.close()
    finally:
        eng.close()
        model.close()


@DTYPES
def test_half_engine_refuses_batched_decode(dtype):
    say(f"{dtype} engine: batched decode is not supported")
    eng = engine(dtype)
    try:
        eng.load_synthetic(1)
        eng.kv_reset(0, 0)
        with pytest.raises(qd.QdError) as err:
            eng.step_batch([0], [3])
        assert err.value.status == qd.NOT_SUPPORTED
    finally:
        eng.close()


@DTYPES
def test_half_resident_equals_stream_at_config2_context(dtype):
    """The full model (24 layers, 151,936-row tied head) with half-width
    decoder weights: a resident generation at context 513..528 (synthetic
    N(0,1) K/V rows) equals the same engine type on its stream-ordered
    kernels (QD_RESIDENT=0) bit for bit: tokens, logits and K/V rows."""
    say(f"{dtype} full model: resident vs stream generation at context 513..528")
    context, steps = 512, 16
    res = qd.Engine(capacity=context + steps + 8, max_batch=1, decoder_dtype=dtype)
    os.environ["QD_RESIDENT"] = "0"
    try:
        stream = qd.Engine(capacity=context + steps + 8, max_batch=1, decoder_dtype=dtype)
    finally:
        del os.environ["QD_RESIDENT"]
    try:
        assert res.resident_grid() > 0 and stream.resident_grid() == 0
        for eng in (res, stream):
            eng.load_synthetic(1)
        for layer in range(24):
            k = qo.fill_normal(context * 128, 7, 0x500000 + 2 * layer, 0.0, 1.0).reshape(context, 128)
            v = qo.fill_normal(context * 128, 7, 0x500000 + 2 * layer + 1, 0.0, 1.0).reshape(context, 128)
            for eng in (res, stream):
                eng.write_kv(0, layer, 0, k, v)
        for eng in (res, stream):
            eng.kv_reset(0, context)
        toks, _, logits = res.generate(0, 31337, steps, want_logits=True)
        toks2, _, logits2 = stream.generate(0, 31337, steps, want_logits=True)
        assert toks.tolist() == toks2.tolist()
        assert np.array_equal(logits, logits2)
        for layer in (0, 11, 23):
            k1, v1 = res.read_kv(0, layer, context, steps)
            k2, v2 = stream.read_kv(0, layer, context, steps)
            assert np.array_equal(k1, k2) and np.array_equal(v1, v2), layer
    finally:
        res.close()
        stream.close()
