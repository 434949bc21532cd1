"""GPU parity of the decode engine against the CPU oracle, through the C ABI.

Bars (from the task's north star):
  * logits: max|gpu - ref| / max|ref| <= 1e-4 (tolerance written below);
  * greedy token identical wherever the oracle's top-1/top-2 margin > 1e-3;
  * argmax index and KV-cache slot indexing bit-exact.
Each test prints the case it runs before touching the GPU.
"""
import os
import sys

import numpy as np
import pytest

import qwen_decode as qd
import qwen_oracle as qo

pytestmark = pytest.mark.gpu

LOGIT_RTOL = 1e-4        # ||delta||_inf / ||ref||_inf on logits
HIDDEN_RTOL = 1e-4       # same norm on hidden states and K/V rows
MARGIN = 1e-3            # top-1/top-2 margin above which tokens must agree
PROMPT_STREAM = 0x300000
HIDDEN_STREAM = 0x100000
KV_STREAM = 0x200000


def say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def rel_err(a, b):
    return float(np.abs(a.astype(np.float64) - b).max() / max(np.abs(b).max(), 1e-30))


def margin(logits):
    top2 = np.partition(logits, -2)[-2:]
    return float(top2[1] - top2[0])


def check_logits(gpu_tok, gpu_logits, ref_tok, ref_logits, what):
    err = rel_err(gpu_logits, ref_logits)
    assert err <= LOGIT_RTOL, f"{what}: logits rel err {err:.3e}"
    # argmax indexing is bit-exact with respect to the engine's own logits
    # (lowest index on ties).
    assert gpu_tok == int(np.argmax(gpu_logits)), what
    if margin(ref_logits) > MARGIN:
        assert gpu_tok == ref_tok, f"{what}: token {gpu_tok} != oracle {ref_tok}"
    return err


# ---- shared full-size model ------------------------------------------------------

FULL = qo.QWEN25_05B
CAPACITY = 5200


@pytest.fixture(scope="module")
def full():
    say("full model: synthetic seed 1, engine + oracle")
    eng = qd.Engine(layers=FULL.layers, vocab=FULL.vocab, capacity=CAPACITY, max_batch=4)
    eng.load_synthetic(1)
    model = qo.Model(FULL)
    model.fill_synthetic(1)
    yield eng, model
    eng.close()
    model.close()


@pytest.fixture(scope="module")
def stream_full():
    """The same model on an engine that generates with the stream-ordered
    kernels only (QD_RESIDENT=0 at create time): the resident kernel's
    bit-exact twin."""
    say("full model: stream-ordered engine (QD_RESIDENT=0)")
    os.environ["QD_RESIDENT"] = "0"
    try:
        eng = qd.Engine(layers=FULL.layers, vocab=FULL.vocab, capacity=CAPACITY, max_batch=2)
    finally:
        del os.environ["QD_RESIDENT"]
    assert eng.resident_grid() == 0
    eng.load_synthetic(1)
    yield eng
    eng.close()


def assert_kv_equal(a, b, slot_a, slot_b, start, count, what):
    """KV rows [start, start + count) of every layer bit-identical."""
    for layer in range(FULL.layers):
        ka, va = a.read_kv(slot_a, layer, start, count)
        kb, vb = b.read_kv(slot_b, layer, start, count)
        assert np.array_equal(ka, kb) and np.array_equal(va, vb), f"{what}: layer {layer}"


def test_synthetic_weights_bit_identical_to_oracle(full):
    eng, model = full
    say("weights readback")
    for layer, kind in [(0, qo.Q_W), (0, qo.K_B), (7, qo.V_W), (23, qo.DOWN_W), (11, qo.GATE_W),
                        (5, qo.ATTN_NORM), (0, qo.FINAL_NORM), (0, qo.EMBED)]:
        ref = model.tensor(layer, kind)
        got = eng.read_weight(layer, kind, ref.size)
        assert np.array_equal(got, ref), (layer, kind)


def test_single_layer_config1():
    """one layer, KV pre-filled to 128 with N(0,1), hidden
    N(0,1), weights seed 0, one step at position 128."""
    say("config1 single layer")
    shape = qo.ModelShape(layers=1, vocab=1024)
    model = qo.Model(shape)
    model.fill_synthetic(0)
    eng = qd.Engine(layers=1, vocab=1024, capacity=256)
    eng.load_synthetic(0)
    k = qo.fill_normal(128 * 128, 0, KV_STREAM, 0.0, 1.0).reshape(128, 128)
    v = qo.fill_normal(128 * 128, 0, KV_STREAM + 1, 0.0, 1.0).reshape(128, 128)
    hidden = qo.fill_normal(896, 0, HIDDEN_STREAM, 0.0, 1.0)
    eng.write_kv(0, 0, 0, k, v)
    eng.kv_reset(0, 128)
    out = eng.layer_step(0, 0, hidden)
    cache = qo.Cache(model, 256)
    cache.layer(0, False)[:128] = k
    cache.layer(0, True)[:128] = v
    ref = cache.layer_step(0, hidden, 128)
    assert rel_err(out, ref) <= HIDDEN_RTOL, rel_err(out, ref)
    gk, gv = eng.read_kv(0, 0, 0, 130)
    # Slots 0..127 untouched, slot 128 written, slot 129 still zero.
    assert np.array_equal(gk[:128], k) and np.array_equal(gv[:128], v)
    assert rel_err(gk[128], cache.layer(0, False)[128]) <= HIDDEN_RTOL
    assert rel_err(gv[128], cache.layer(0, True)[128]) <= HIDDEN_RTOL
    assert not gk[129].any() and not gv[129].any()
    # The layer step does not advance the slot.
    assert eng.decode_state(0).token_position == 128
    eng.close()


def test_full_model_prefill_and_decode(full):
    eng, model = full
    prompt = qo.fill_tokens(8, 1, PROMPT_STREAM, FULL.vocab)
    say(f"full model prefill {prompt.tolist()} + 8 teacher-forced steps")
    eng.kv_reset(0, 0)
    cache = qo.Cache(model, 64)
    tok, top, logits = eng.prefill(0, prompt)
    rtok, rtop, rlogits = cache.prefill(prompt)
    errs = [check_logits(tok, logits, rtok, rlogits, "prefill")]
    assert abs(top - logits[tok]) == 0.0
    feed = rtok
    for i in range(8):
        pos = len(prompt) + i
        tok, top, logits = eng.step(0, feed)
        rtok, rtop, rlogits = cache.decode_step(feed, pos)
        errs.append(check_logits(tok, logits, rtok, rlogits, f"step {i}"))
        feed = rtok
    say(f"max logits rel err {max(errs):.3e}")
    assert eng.decode_state(0).token_position == len(prompt) + 8
    # KV cache rows (post-RoPE K, raw V) at every written slot of two layers.
    for layer in (0, 23):
        gk, gv = eng.read_kv(0, layer, 0, 16)
        assert rel_err(gk, cache.layer(layer, False)[:16]) <= HIDDEN_RTOL
        assert rel_err(gv, cache.layer(layer, True)[:16]) <= HIDDEN_RTOL
        tail_k, _ = eng.read_kv(0, layer, 16, 4)
        assert not tail_k.any()


def test_generate_matches_step_loop_and_oracle(full):
    eng, model = full
    prompt = qo.fill_tokens(6, 1, PROMPT_STREAM + 1, FULL.vocab)
    say("generate vs step loop vs oracle greedy chain")
    # Step loop on slot 1.
    eng.kv_reset(1, 0)
    first, _, _ = eng.prefill(1, prompt, want_logits=False)
    steps, step_logits, feed = [], [], first
    for _ in range(6):
        feed, _, lg = eng.step(1, feed)
        steps.append(feed)
        step_logits.append(lg)
    # Device-resident generation on slot 2 from the same prefix.
    eng.kv_reset(2, 0)
    first2, _, _ = eng.prefill(2, prompt, want_logits=False)
    assert first2 == first
    toks, reason, gen_logits = eng.generate(2, first, 6, want_logits=True)
    assert reason == qd.STOP_MAXIMUM_TOKENS
    assert toks.tolist() == steps
    # Same kernels, same inputs: the two paths are bit-identical.
    assert np.array_equal(gen_logits, np.stack(step_logits))
    assert eng.decode_state(2).token_position == len(prompt) + 6
    # Oracle greedy chain: identical until the first low-margin step.
    cache = qo.Cache(model, 64)
    rtok, _, rlog = cache.prefill(prompt)
    assert rtok == first or margin(rlog) <= MARGIN
    feed = rtok
    for i, t in enumerate(toks.tolist()):
        rtok, _, rlog = cache.decode_step(feed, len(prompt) + i)
        check_logits(t, gen_logits[i], rtok, rlog, f"generate step {i}")
        if margin(rlog) <= MARGIN:
            break
        feed = rtok


def test_resident_and_stream_generation_agree(full, stream_full):
    """The resident megakernel and the stream-ordered kernels run the same
    arithmetic in the same order: identical tokens, logits and KV rows."""
    eng, _ = full
    assert eng.resident_grid() > 0
    prompt = qo.fill_tokens(9, 1, PROMPT_STREAM + 3, FULL.vocab)
    say("resident vs stream generation, 12 tokens")
    eng.kv_reset(0, 0)
    first, _, _ = eng.prefill(0, prompt, want_logits=False)
    toks, _, logits = eng.generate(0, first, 12, want_logits=True)
    stream = stream_full
    stream.kv_reset(0, 0)
    first2, _, _ = stream.prefill(0, prompt, want_logits=False)
    toks2, _, logits2 = stream.generate(0, first2, 12, want_logits=True)
    assert first2 == first and toks2.tolist() == toks.tolist()
    assert np.array_equal(logits, logits2)
    # KV rows written by the resident launch (the last token's included).
    assert_kv_equal(eng, stream, 0, 0, len(prompt), 12, "resident KV")


def test_resident_across_chunk_length_changes_matches_stream(full, stream_full):
    """Attention chunks are whole multiples of 16 positions split over the engine's
    attention parts (9 on a 256-CU MI355X): across context 1001..1170 the
    chunk length grows from 112 to 128 positions at 1009 and to 144 at 1153,
    and the chunk count drops from 9 to 8 at 1009 and regrows to 9 at 1025.
    A resident generation across these points equals the stream path bit
    for bit (hand-off slots beyond the chunk count hold older records)."""
    eng, _ = full
    prompt = qo.fill_tokens(1000, 1, PROMPT_STREAM + 4, FULL.vocab)
    say("resident vs stream generation, context 1001..1170")
    eng.kv_reset(1, 0)
    first, _, _ = eng.prefill(1, prompt, want_logits=False)
    toks, _, logits = eng.generate(1, first, 170, want_logits=True)
    stream = stream_full
    stream.kv_reset(0, 0)
    first2, _, _ = stream.prefill(0, prompt, want_logits=False)
    toks2, _, logits2 = stream.generate(0, first2, 170, want_logits=True)
    assert first2 == first and toks2.tolist() == toks.tolist()
    assert np.array_equal(logits, logits2)
    assert_kv_equal(eng, stream, 1, 0, len(prompt), 170, "resident KV")


def synthetic_context(engines, cache, length, seed=7):
    """N(0,1) K/V rows at positions [0, length) of every layer, written into
    slot 0 of each engine and into the oracle cache."""
    for layer in range(FULL.layers):
        k = qo.fill_normal(length * 128, seed, KV_STREAM + 2 * layer, 0.0, 1.0).reshape(length, 128)
        v = qo.fill_normal(length * 128, seed, KV_STREAM + 2 * layer + 1, 0.0, 1.0).reshape(length, 128)
        for e in engines:
            e.write_kv(0, layer, 0, k, v)
        cache.layer(layer, False)[:length] = k
        cache.layer(layer, True)[:length] = v
    for e in engines:
        e.kv_reset(0, length)


def long_context_generation(full, stream_full, context, steps, token, what):
    """Resident generation of `steps` tokens after a synthetic context,
    against the stream path (bit-exact tokens, logits, KV rows) and the
    oracle teacher-forced on the engine's tokens (logits within the bar)."""
    eng, model = full
    cache = qo.Cache(model, context + steps + 8)
    synthetic_context([eng, stream_full], cache, context)
    say(f"{what}: resident generation")
    toks, reason, logits = eng.generate(0, token, steps, want_logits=True)
    assert reason == qd.STOP_MAXIMUM_TOKENS and len(toks) == steps
    say(f"{what}: stream generation")
    toks2, _, logits2 = stream_full.generate(0, token, steps, want_logits=True)
    assert toks.tolist() == toks2.tolist()
    assert np.array_equal(logits, logits2)
    assert_kv_equal(eng, stream_full, 0, 0, context, steps, what)
    say(f"{what}: oracle, {steps} teacher-forced steps")
    feed, errs = token, []
    for i in range(steps):
        last = i == steps - 1
        want = last or i % 8 == 0
        rtok, _, rlog = cache.decode_step(feed, context + i, want_logits=want)
        if want:
            errs.append(check_logits(int(toks[i]), logits[i], rtok, rlog, f"{what} step {i}"))
        feed = int(toks[i])
    gk, gv = eng.read_kv(0, 23, context + steps - 1, 1)
    assert rel_err(gk[0], cache.layer(23, False)[context + steps - 1]) <= HIDDEN_RTOL
    assert rel_err(gv[0], cache.layer(23, True)[context + steps - 1]) <= HIDDEN_RTOL
    cache.close()
    say(f"{what}: max logits rel err {max(errs):.3e}")


def test_resident_config2_context_512_matches_stream_and_oracle(full, stream_full):
    """BASELINE config 2's range as the bench runs it: the resident kernel at
    context 513..528 (9 chunks of 64 positions per KV head), against the
    stream path bit for bit and the oracle."""
    long_context_generation(full, stream_full, 512, 16, 31337, "config 2 resident 513..528")


def test_config2_bench_chain_matches_oracle(full):
    """BASELINE config 2 exactly as bench.py runs it: the seed-1 model, the
    512-token prompt of the bench's stream prefilled on the MFMA path, then
    one resident launch of 64 greedy tokens (context 513..576). Every step's
    logits and token against the oracle teacher-forced on the engine's
    tokens."""
    eng, model = full
    prompt = qo.fill_tokens(512, 1, PROMPT_STREAM, FULL.vocab)
    say("config 2 bench chain: prefill 512 + 64 resident tokens vs oracle")
    eng.kv_reset(3, 0)
    first, _, _ = eng.prefill(3, prompt, want_logits=False)
    toks, reason, logits = eng.generate(3, first, 64, want_logits=True)
    assert reason == qd.STOP_MAXIMUM_TOKENS and len(toks) == 64
    cache = qo.Cache(model, 512 + 64 + 8)
    rtok, _, rlog = cache.prefill(prompt)
    assert rtok == first or margin(rlog) <= MARGIN
    feed, errs = first, []
    for i, t in enumerate(toks.tolist()):
        rtok, _, rlog = cache.decode_step(feed, 512 + i)
        errs.append(check_logits(t, logits[i], rtok, rlog, f"config 2 step {i}"))
        feed = t
    gk, gv = eng.read_kv(3, 23, 512, 64)
    assert rel_err(gk, cache.layer(23, False)[512:576]) <= HIDDEN_RTOL
    assert rel_err(gv, cache.layer(23, True)[512:576]) <= HIDDEN_RTOL
    cache.close()
    say(f"config 2 bench chain: max logits rel err {max(errs):.3e}")


def test_resident_config3_context_4096_matches_stream_and_oracle(full, stream_full):
    """BASELINE config 3 as the bench runs it: the resident kernel at context
    4065..4096 (on a 256-CU MI355X, 464-position chunks, 9 per KV head, each
    walked in two windows, the first in LDS and the second in the waves'
    registers, its 32-position tiles spread over the waves on MFMA)."""
    long_context_generation(full, stream_full, 4064, 32, 4242, "config 3 resident 4065..4096")


def test_resident_multi_window_beyond_4096_matches_stream_and_oracle(full, stream_full):
    """Across context 4096 (4091..4130; 464-position chunks, 9 per KV head,
    on a 256-CU MI355X), each chunk walked in two windows: 256 positions in
    LDS, then the rest in the waves' registers."""
    long_context_generation(full, stream_full, 4090, 40, 777, "resident 4091..4130 (two windows)")


def test_resident_third_window_beyond_4608_matches_stream_and_oracle(full, stream_full):
    """Above context 4608 (5101..5130; 576-position chunks on a 256-CU
    MI355X) a chunk needs a third window: after the LDS window and the
    register window, the last positions are loaded into LDS again."""
    long_context_generation(full, stream_full, 5100, 30, 999, "resident 5101..5130 (three windows)")


def test_resident_step_and_graph_agree(full):
    """The reference's three-way cross-check of one greedy chain
    (benchmarks/qwen_stateful_graph.cpp:1619-1746): the resident megakernel
    over several tokens (qd_generate_resident), one resident launch per token
    (qd_step) and the stream-ordered step kernels replayed from a captured
    HIP graph (qd_step_graph, one graph per slot,
    benchmarks/qwen_hip_graph.hpp:27-199) give the same tokens, logits, top
    logits, positions and K/V rows, bit for bit. Every graph replay is
    checked against the step that ran just before it, with the program's
    own work and host synchronisations in between."""
    eng, _ = full
    prompt = qo.fill_tokens(11, 1, PROMPT_STREAM + 9, FULL.vocab)
    steps = 8
    say("resident vs qd_step vs qd_step_graph, 8 greedy tokens")
    firsts = []
    for slot in (0, 1, 2):
        eng.kv_reset(slot, 0)
        t, _, _ = eng.prefill(slot, prompt, want_logits=False)
        firsts.append(t)
    assert firsts[0] == firsts[1] == firsts[2]
    rtoks, _, rlogits = eng.generate(0, firsts[0], steps, want_logits=True)
    fs = fg = firsts[0]
    for i in range(steps):
        ts, tops, ls = eng.step(1, fs)
        tg, topg, lg = eng.step_graph(2, fg)
        assert ts == tg == int(rtoks[i]) and tops == topg, i
        assert np.array_equal(ls, lg) and np.array_equal(ls, rlogits[i]), i
        assert eng.decode_state(1).token_position == eng.decode_state(2).token_position == len(prompt) + i + 1
        # qd_step's one-token resident launch leaves the stream step's state.
        d1, d2 = eng.decode_state(1), eng.decode_state(2)
        assert [getattr(d1, f) for f, _ in qd.DecodeState._fields_] == \
            [getattr(d2, f) for f, _ in qd.DecodeState._fields_], i
        fs, fg = ts, tg
    assert_kv_equal(eng, eng, 0, 1, len(prompt), steps, "resident vs step KV")
    assert_kv_equal(eng, eng, 1, 2, len(prompt), steps, "step vs graph KV")
    assert np.array_equal(eng.read_logits(2), rlogits[-1])
    # A resident launch right after graph replays on the same stream: the
    # dispatcher may start it from another XCD than 0, and the kernel's
    # placement follows the XCD each workgroup runs on.
    eng.kv_reset(0, len(prompt))
    rtoks2, _, rlogits2 = eng.generate(0, firsts[0], steps, want_logits=True)
    assert np.array_equal(rtoks2, rtoks) and np.array_equal(rlogits2, rlogits)


def test_layer_by_layer_decode_equals_step(full):
    """The reference driver's per-token loop through the C ABI
    (benchmarks/triton_mini_decoder_layer.cpp:1051-1068): the embedding row
    into the slot's hidden, 24 device hand-offs (qd_layer_decode, one layer
    per call: decode_to_hidden_state / decode_to_buffer), then qd_tail
    (ModelTail::run) gives qd_step's token, logits and K/V rows bit for bit;
    so does one call for the whole stack after a host-side embedding row."""
    eng, _ = full
    prompt = qo.fill_tokens(7, 1, PROMPT_STREAM + 6, FULL.vocab)
    say("layer-by-layer decode vs qd_step, 4 tokens")
    for slot in (0, 1):
        eng.kv_reset(slot, 0)
        first, _, _ = eng.prefill(slot, prompt, want_logits=False)
    emb = eng.read_weight(0, qd.EMBED, FULL.vocab * FULL.hidden).reshape(FULL.vocab, FULL.hidden)
    feed = first
    for i in range(4):
        pos = len(prompt) + i
        tok, top, logits = eng.step(0, feed)
        if i % 2 == 0:
            eng.embed_hidden(1, feed)
            for layer in range(FULL.layers):
                eng.layer_decode(1, layer, 1, pos + 1)
        else:
            eng.load_hidden(1, emb[feed])
            eng.layer_decode(1, 0, FULL.layers, pos + 1)
        tok2, top2, logits2 = eng.tail(1)
        assert tok2 == tok and top2 == top, i
        assert np.array_equal(logits2, logits), i
        assert np.array_equal(eng.read_logits(1), logits), i
        assert eng.decode_state(1).token_position == pos + 1
        feed = tok
    assert_kv_equal(eng, eng, 0, 1, len(prompt), 4, "layer-by-layer KV")
    # The slot continues with the fused path from where the layers left it.
    a, _, la = eng.step(0, feed)
    b, _, lb = eng.step(1, feed)
    assert a == b and np.array_equal(la, lb)


def test_generate_stops_at_eos(full):
    eng, _ = full
    prompt = qo.fill_tokens(5, 1, PROMPT_STREAM + 2, FULL.vocab)
    say("eos stop")
    eng.kv_reset(3, 0)
    first, _, _ = eng.prefill(3, prompt, want_logits=False)
    toks, reason, _ = eng.generate(3, first, 5)
    assert reason == qd.STOP_MAXIMUM_TOKENS and len(toks) == 5
    eos = int(toks[2])
    if eos in toks[:2].tolist():
        pytest.skip("EOS candidate repeats earlier in the chain")
    eng.kv_reset(3, len(prompt))
    toks2, reason2, _ = eng.generate(3, first, 5, eos=eos)
    assert reason2 == qd.STOP_EOS_TOKEN
    assert toks2.tolist() == toks[:3].tolist()
    st = eng.decode_state(3)
    assert st.generated_tokens == 3 and st.stop_reason == qd.STOP_EOS_TOKEN
    assert st.token_position == len(prompt) + 3


def test_batch_step_matches_oracle_per_sequence(full):
    eng, model = full
    say("step_batch over 3 ragged sequences")
    prompts = [qo.fill_tokens(n, 1, PROMPT_STREAM + 10 + i, FULL.vocab) for i, n in enumerate((3, 7, 5))]
    caches, feeds = [], []
    for slot, p in enumerate(prompts):
        eng.kv_reset(slot, 0)
        eng.prefill(slot, p, want_logits=False)
        c = qo.Cache(model, 16)
        c.prefill(p, want_logits=False)
        caches.append(c)
        feeds.append(int(p[0]))
    greedy, logits = eng.step_batch([0, 1, 2], feeds)
    for slot, p in enumerate(prompts):
        rtok, _, rlog = caches[slot].decode_step(feeds[slot], len(p))
        check_logits(int(greedy[slot]), logits[slot], rtok, rlog, f"batch seq {slot}")


def test_prefill_512_config5_matches_oracle():
    """BASELINE config 5 on its own model (weights seed 4): the 512-token
    prompt through the MFMA prompt path (dense GEMMs + causal attention),
    then 128 greedy decode steps reusing its cache: 3 qd_step calls, the rest
    one resident generation, each against the oracle teacher-forced on the
    engine's tokens."""
    say("config 5: seed-4 model, engine + oracle")
    eng = qd.Engine(layers=FULL.layers, vocab=FULL.vocab, capacity=512 + 128 + 8, max_batch=1)
    eng.load_synthetic(4)
    model = qo.Model(FULL)
    model.fill_synthetic(4)
    try:
        prompt = qo.fill_tokens(512, 4, PROMPT_STREAM, FULL.vocab)
        say("prefill 512 (config 5) vs oracle")
        eng.kv_reset(0, 0)
        cache = qo.Cache(model, 530 + 128)
        tok, _, logits = eng.prefill(0, prompt)
        rtok, _, rlogits = cache.prefill(prompt)
        check_logits(tok, logits, rtok, rlogits, "prefill 512")
        assert eng.decode_state(0).token_position == 512
        for layer in (0, 11, 23):
            gk, gv = eng.read_kv(0, layer, 0, 512)
            assert rel_err(gk, cache.layer(layer, False)[:512]) <= HIDDEN_RTOL, layer
            assert rel_err(gv, cache.layer(layer, True)[:512]) <= HIDDEN_RTOL, layer
        feed = tok
        for i in range(3):
            tok, _, logits = eng.step(0, feed)
            rtok, _, rlogits = cache.decode_step(feed, 512 + i)
            check_logits(tok, logits, rtok, rlogits, f"decode after prefill {i}")
            feed = tok
        say("resident generation of the other 125 steps (context 516..640) vs oracle")
        toks, reason, gen_logits = eng.generate(0, feed, 125, want_logits=True)
        assert reason == qd.STOP_MAXIMUM_TOKENS and len(toks) == 125
        errs = []
        for i, t in enumerate(toks.tolist()):
            rtok, _, rlogits = cache.decode_step(feed, 515 + i)
            errs.append(check_logits(t, gen_logits[i], rtok, rlogits, f"resident after prefill {i}"))
            feed = t
        gk, gv = eng.read_kv(0, 23, 639, 1)
        assert rel_err(gk[0], cache.layer(23, False)[639]) <= HIDDEN_RTOL
        assert rel_err(gv[0], cache.layer(23, True)[639]) <= HIDDEN_RTOL
        say(f"config 5: max logits rel err {max(errs):.3e}")
        cache.close()
    finally:
        eng.close()
        model.close()


def test_profile_prefill_matches_prefill(full):
    """qd_profile_prefill times the prompt kernels by projection and leaves
    the slot exactly as qd_prefill does (same kernels: bit-identical KV)."""
    eng, _ = full
    prompt = qo.fill_tokens(96, 4, PROMPT_STREAM + 3, FULL.vocab)
    say("profile_prefill vs prefill, 96 tokens")
    eng.kv_reset(0, 0)
    eng.kv_reset(1, 0)
    prof = eng.profile_prefill(0, prompt)
    tok, _, _ = eng.prefill(1, prompt, want_logits=False)
    assert eng.decode_state(0).token_position == 96
    assert eng.decode_state(0).sampled_token == tok
    for layer in (0, 23):
        k0, v0 = eng.read_kv(0, layer, 0, 96)
        k1, v1 = eng.read_kv(1, layer, 0, 96)
        assert np.array_equal(k0, k1) and np.array_equal(v0, v1), layer
    h, i, qkv = FULL.hidden, FULL.intermediate, (FULL.heads + 2 * FULL.kv_heads) * FULL.head_dim
    expect = {"gemm_nt_kernel:qkv+rope": 2 * 96 * qkv * h, "gemm_nt_kernel:gateup+swiglu": 4 * 96 * i * h,
              "gemm_nt_kernel:down+norm": 2 * 96 * h * i}
    for name, flops in expect.items():
        launches, avg_us, _, avg_flops = prof[name]
        assert launches == FULL.layers and avg_us > 0 and avg_flops == flops, name
    assert prof["lmhead_kernel+argmax"][0] == 1


def test_prefill_in_pieces_and_over_chunks_agree(full):
    """A prompt prefilled in two calls (the second continuing at position 300)
    and one longer than a 512-row chunk give the one-call results."""
    eng, _ = full
    prompt = qo.fill_tokens(700, 4, PROMPT_STREAM + 5, FULL.vocab)
    say("prefill 700 at once / 300 + 400")
    eng.kv_reset(0, 0)
    tok, _, logits = eng.prefill(0, prompt)
    k_once, v_once = eng.read_kv(0, 5, 0, 700)
    eng.kv_reset(1, 0)
    eng.prefill(1, prompt[:300], want_logits=False)
    tok2, _, logits2 = eng.prefill(1, prompt[300:])
    assert eng.decode_state(1).token_position == 700
    assert tok2 == tok or margin(logits) <= MARGIN
    assert rel_err(logits2, logits) <= LOGIT_RTOL
    k_two, v_two = eng.read_kv(1, 5, 0, 700)
    assert rel_err(k_two, k_once) <= HIDDEN_RTOL and rel_err(v_two, v_once) <= HIDDEN_RTOL


def test_long_context_4096(full):
    """BASELINE config 3 attention length: one step at position 4096 over a
    synthetic N(0,1) KV cache in every layer."""
    eng, model = full
    say("context 4096 step")
    L = 4096
    cache = qo.Cache(model, L + 8)
    for layer in range(FULL.layers):
        k = qo.fill_normal(L * 128, 7, KV_STREAM + 2 * layer, 0.0, 1.0).reshape(L, 128)
        v = qo.fill_normal(L * 128, 7, KV_STREAM + 2 * layer + 1, 0.0, 1.0).reshape(L, 128)
        eng.write_kv(0, layer, 0, k, v)
        cache.layer(layer, False)[:L] = k
        cache.layer(layer, True)[:L] = v
    eng.kv_reset(0, L)
    token = 4242
    tok, _, logits = eng.step(0, token)
    rtok, _, rlog = cache.decode_step(token, L)
    err = check_logits(tok, logits, rtok, rlog, "context 4096")
    say(f"context 4096 logits rel err {err:.3e}")
    gk, gv = eng.read_kv(0, 12, L, 1)
    assert rel_err(gk[0], cache.layer(12, False)[L]) <= HIDDEN_RTOL


def test_argument_errors_do_not_touch_the_device(full):
    eng, _ = full
    say("argument validation")
    with pytest.raises(qd.QdError) as e:
        eng.step(0, FULL.vocab)
    assert e.value.status == qd.INVALID_ARGUMENT
    with pytest.raises(qd.QdError):
        eng.kv_reset(9, 0)
    eng.kv_reset(0, CAPACITY)
    with pytest.raises(qd.QdError) as e:
        eng.step(0, 1)
    assert "full" in str(e.value)
    with pytest.raises(qd.QdError):
        eng.step_batch([0, 0], [1, 2])
