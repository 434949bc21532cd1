"""Failure handling of the engine on the GPU, forced from the host.

* A resident hand-off wait that exhausts its spin limit ends the launch with
  QD_ERROR_DEVICE_FAULT and a message that says so; every workgroup exits
  (the call returns) and the engine keeps working. The give-up is forced
  with QD_RESIDENT_SPIN_LIMIT=1 at engine creation: waits then give up after
  a few polls, long before any producer publishes.
* NaN payloads never survive a load: K/V rows written through qd_write_kv
  and weights loaded from a bundle hold only the canonical NaN 0x7FC00000,
  so a NaN whose bits equal the resident kernel's empty-slot pattern
  (0xFFFFFFFF) cannot stall a hand-off; a NaN model decodes to NaN logits on
  the resident path without waiting.
"""
import os

import numpy as np
import pytest

import qwen_decode as qd
import qwen_oracle as qo

pytestmark = pytest.mark.gpu

SMALL = dict(layers=2, vocab=4096, capacity=64, max_batch=1)
CANONICAL = 0x7FC00000


def say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def test_resident_wait_give_up_reports_device_fault(monkeypatch):
    say("resident wait give-up: QD_RESIDENT_SPIN_LIMIT=1")
    monkeypatch.setenv("QD_RESIDENT_SPIN_LIMIT", "1")
    eng = qd.Engine(**SMALL)
    monkeypatch.delenv("QD_RESIDENT_SPIN_LIMIT")
    ref = qd.Engine(**SMALL)
    try:
        assert eng.resident_grid() > 0
        for e in (eng, ref):
            e.load_synthetic(5)
        prompt = qo.fill_tokens(4, 5, 0x300000, SMALL["vocab"])
        eng.kv_reset(0, 0)
        first, _, _ = eng.prefill(0, prompt, want_logits=False)
        with pytest.raises(qd.QdError) as err:
            eng.generate(0, first, 4)
        assert err.value.status == qd.DEVICE_FAULT
        assert "gave up" in str(err.value)
        # The position did not move, and the device is healthy: a stream step
        # (the graph replay of the step kernels) from the same state equals
        # the step on an untouched engine (the resident kernel's one-token
        # launch, as qd_step runs it there).
        assert eng.decode_state(0).token_position == len(prompt)
        ref.kv_reset(0, 0)
        ref.prefill(0, prompt, want_logits=False)
        tok, _, logits = eng.step_graph(0, first)
        tok2, _, logits2 = ref.step(0, first)
        assert tok == tok2 and np.array_equal(logits, logits2)
        # And the untouched engine's resident path still completes.
        toks, reason, _ = ref.generate(0, tok2, 3)
        assert reason == qd.STOP_MAXIMUM_TOKENS and len(toks) == 3
    finally:
        eng.close()
        ref.close()


def nan_bits(*patterns):
    return np.array(patterns, np.uint32).view(np.float32)


def test_write_kv_canonicalises_nan():
    say("write_kv NaN payloads")
    eng = qd.Engine(**SMALL)
    try:
        k = qo.fill_normal(8 * 128, 3, 0x200000, 0.0, 1.0).reshape(8, 128)
        v = qo.fill_normal(8 * 128, 3, 0x200001, 0.0, 1.0).reshape(8, 128)
        k[1, 5], k[7, 127] = nan_bits(0xFFFFFFFF, 0x7FFFFFFF)
        v[0, 0], v[3, 64] = nan_bits(0xFFC00001, 0x7F800001)
        eng.write_kv(0, 1, 10, k, v)
        gk, gv = eng.read_kv(0, 1, 10, 8)
        for got, want in ((gk, k), (gv, v)):
            nan = np.isnan(want)
            assert np.array_equal(np.isnan(got), nan)
            assert (got.view(np.uint32)[nan] == CANONICAL).all()
            assert np.array_equal(got.view(np.uint32)[~nan], want.view(np.uint32)[~nan])
    finally:
        eng.close()


def test_bundle_nan_weights_are_canonical_and_resident_decode_returns(tmp_path):
    say("bundle with NaN payloads: load, canonical NaN, resident decode returns")
    h, i, q, kv, vocab = 896, 4864, 896, 128, 1024
    sizes = [h, h, q * h, kv * h, kv * h, q, kv, kv, h * q, i * h, i * h, h * i]
    tensors = [qo.fill_normal(n, 9, 0x400000 + j, 0.0, 0.02) for j, n in enumerate(sizes)]
    tensors[0][:] = 1.0
    tensors[1][:] = 1.0
    tensors[2][0] = nan_bits(0xFFFFFFFF)[0]   # q weight
    tensors[9][5] = nan_bits(0x7FFFFFFF)[0]   # gate weight
    tensors[11][-1] = nan_bits(0xFFC00001)[0]  # down weight
    layer_dir = tmp_path / "layer_0"
    layer_dir.mkdir()
    qd.bundle_write_layer(str(layer_dir / "weights.json"), "weights.bin", [1, h, 14, 2, 64, i], 1e6,
                          np.concatenate(tensors))
    emb = qo.fill_normal(vocab * h, 9, 0x500000, 0.0, 0.02)
    emb[3] = nan_bits(0xFFFFFFFF)[0]
    tail_dir = tmp_path / "model_tail"
    tail_dir.mkdir()
    qd.bundle_write_tail(str(tail_dir / "weights.json"), "weights.bin", h, vocab, np.arange(vocab),
                         emb, np.ones(h, np.float32), emb)
    eng = qd.Engine(layers=1, vocab=vocab, capacity=32, max_batch=1)
    try:
        eng.load_bundle(str(tmp_path))
        for kind, idx in ((qo.Q_W, 0), (qo.GATE_W, 5), (qo.DOWN_W, sizes[11] - 1)):
            got = eng.read_weight(0, kind, sizes[kind])
            assert got.view(np.uint32)[idx] == CANONICAL, kind
            assert np.isnan(got).sum() == 1, kind
        assert eng.read_weight(0, qd.EMBED, vocab * h).view(np.uint32)[3] == CANONICAL
        # Every hidden state is NaN from the first layer on (the NaN query
        # weight reaches every head through the O projection): the resident
        # launch must still run to its end and report a NaN argmax.
        assert eng.resident_grid() > 0
        eng.kv_reset(0, 0)
        toks, reason, logits = eng.generate(0, 7, 3, want_logits=True)
        assert toks.tolist() == [0xFFFFFFFF] and reason == qd.STOP_NONE
        assert np.isnan(logits).all()
    finally:
        eng.close()
