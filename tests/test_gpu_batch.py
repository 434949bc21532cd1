"""Batched ragged decode through the C ABI on the GPU.

Sixteen sequences with contexts drawn uniformly from [256, 2048] (seed 3)
take greedy steps together through qd_step_batch, whose projections are
skinny M=16 GEMMs on the FP32 matrix cores. Parity:
  * each batched step of every sequence against the batch-1 step of the same
    sequence from the same cache state (the batch-1 path is pinned against
    the oracle in test_gpu_decode.py);
  * the two shortest sequences directly against the CPU oracle, and all 16
    (up to context 2,048) against the oracle decoding over the engine's own
    K/V rows;
  * KV-cache slot indexing: the step writes exactly row L of each slot's
    cache, rows below L stay bit-identical, and row L matches the oracle's.
Bars as in test_gpu_decode.py: logits max|d|/max|ref| <= 1e-4, tokens equal
where the reference's top-1/top-2 margin exceeds 1e-3.
"""
import numpy as np
import pytest

import qwen_decode as qd
import qwen_oracle as qo

pytestmark = pytest.mark.gpu

LOGIT_RTOL = 1e-4
HIDDEN_RTOL = 1e-4
MARGIN = 1e-3
SEED = 3
ROWS = 16
STEPS = 32
LEN_STREAM = 0x400000
PROMPT_STREAM = 0x410000
SHAPE = qo.QWEN25_05B
CAPACITY = 2048 + STEPS + 8


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
    assert gpu_tok == int(np.argmax(gpu_logits)), what
    if margin(ref_logits) > MARGIN:
        assert gpu_tok == ref_tok, f"{what}: token {gpu_tok} != reference {ref_tok}"


def config4_lengths():
    """Contexts uniform in [256, 2048] from the shared counter-based generator."""
    return [256 + int(x) for x in qo.fill_tokens(ROWS, SEED, LEN_STREAM, 2048 - 256 + 1)]


@pytest.fixture(scope="module")
def batch16():
    say("config 4 engine: synthetic seed 3, 16 slots, MFMA prefill of ragged prompts")
    eng = qd.Engine(layers=SHAPE.layers, vocab=SHAPE.vocab, capacity=CAPACITY, max_batch=ROWS + 2)
    eng.load_synthetic(SEED)
    lengths = config4_lengths()
    prompts = [qo.fill_tokens(n, SEED, PROMPT_STREAM + i, SHAPE.vocab) for i, n in enumerate(lengths)]
    firsts = []
    for slot, p in enumerate(prompts):
        eng.kv_reset(slot, 0)
        tok, _, _ = eng.prefill(slot, p, want_logits=False)
        firsts.append(tok)
    yield eng, lengths, prompts, firsts
    eng.close()


def test_config4_lengths_are_ragged_in_range():
    lengths = config4_lengths()
    assert all(256 <= n <= 2048 for n in lengths)
    assert len(set(lengths)) > 8


def test_batch16_first_step_matches_oracle_and_single_steps(batch16):
    eng, lengths, prompts, firsts = batch16
    slots = list(range(ROWS))
    before = {s: eng.read_kv(s, 5, 0, lengths[s]) for s in (0, 7, 15)}
    say("batch step over 16 ragged sequences")
    greedy, logits = eng.step_batch(slots, firsts)
    for s in slots:
        assert eng.decode_state(s).token_position == lengths[s] + 1
        assert int(greedy[s]) == int(np.argmax(logits[s])), s
    # Rows below each sequence's length are untouched; row L is this step's.
    batch_kv = {}
    for s, (k0, v0) in before.items():
        k1, v1 = eng.read_kv(s, 5, 0, lengths[s] + 1)
        assert np.array_equal(k1[:-1], k0) and np.array_equal(v1[:-1], v0), s
        batch_kv[s] = (k1[-1].copy(), v1[-1].copy())
    # The two shortest sequences against the CPU oracle.
    model = qo.Model(SHAPE)
    model.fill_synthetic(SEED)
    try:
        for s in sorted(slots, key=lambda i: lengths[i])[:2]:
            say(f"oracle: slot {s}, context {lengths[s]}")
            cache = qo.Cache(model, lengths[s] + 4)
            rtok, _, _ = cache.prefill(prompts[s], want_logits=False)
            assert rtok == firsts[s], s
            rtok, _, rlog = cache.decode_step(firsts[s], lengths[s])
            check_logits(int(greedy[s]), logits[s], rtok, rlog, f"batch slot {s} vs oracle")
            k, v = eng.read_kv(s, 5, lengths[s], 1)
            assert rel_err(k[0], cache.layer(5, False)[lengths[s]]) <= HIDDEN_RTOL, s
            assert rel_err(v[0], cache.layer(5, True)[lengths[s]]) <= HIDDEN_RTOL, s
            cache.close()
    finally:
        model.close()
    # Every sequence against the batch-1 step from the same cache state.
    say("batch-1 steps of the same positions")
    for s in slots:
        eng.kv_reset(s, lengths[s])
        tok, _, single = eng.step(s, firsts[s])
        check_logits(int(greedy[s]), logits[s], tok, single, f"batch vs single, slot {s}")
        if s in batch_kv:
            k, v = eng.read_kv(s, 5, lengths[s], 1)
            assert rel_err(batch_kv[s][0], k[0]) <= HIDDEN_RTOL, s
            assert rel_err(batch_kv[s][1], v[0]) <= HIDDEN_RTOL, s


def test_batch16_every_sequence_matches_oracle_on_engine_kv(batch16):
    """One batched step of all 16 sequences, each against the CPU oracle
    decoding the same token at the same position over the engine's own K/V
    rows [0, L) (read back through qd_read_kv and written into the oracle's
    cache), so the longest contexts (up to 2,048) are checked directly, not
    only through the batch-1 path. The batched logits also stay on the
    device in each slot's row (qd_read_logits)."""
    eng, lengths, prompts, firsts = batch16
    slots = list(range(ROWS))
    for s in slots:
        eng.kv_reset(s, lengths[s])
    say("batch step over 16 ragged sequences")
    greedy, logits = eng.step_batch(slots, firsts)
    for s in slots:
        assert np.array_equal(eng.read_logits(s), logits[s]), s
    model = qo.Model(SHAPE)
    model.fill_synthetic(SEED)
    try:
        for s in sorted(slots, key=lambda i: -lengths[i]):
            say(f"oracle over the engine's K/V: slot {s}, context {lengths[s]}")
            cache = qo.Cache(model, lengths[s] + 4)
            for layer in range(SHAPE.layers):
                k, v = eng.read_kv(s, layer, 0, lengths[s])
                cache.layer(layer, False)[: lengths[s]] = k
                cache.layer(layer, True)[: lengths[s]] = v
            rtok, _, rlog = cache.decode_step(firsts[s], lengths[s])
            check_logits(int(greedy[s]), logits[s], rtok, rlog, f"batch slot {s} (context {lengths[s]}) vs oracle")
            k, v = eng.read_kv(s, 11, lengths[s], 1)
            assert rel_err(k[0], cache.layer(11, False)[lengths[s]]) <= HIDDEN_RTOL, s
            assert rel_err(v[0], cache.layer(11, True)[lengths[s]]) <= HIDDEN_RTOL, s
            cache.close()
    finally:
        model.close()


def test_batch_step_leaves_other_slots_logits(batch16):
    """qd_read_logits returns each slot's logits of its last step: a batched
    step over other slots leaves a slot's qd_tail logits in place."""
    eng, lengths, _, firsts = batch16
    say("qd_tail on slot 0, then a batched step of slots 1..15")
    eng.kv_reset(0, lengths[0])
    eng.embed_hidden(0, firsts[0])
    eng.layer_decode(0, 0, SHAPE.layers, lengths[0] + 1)
    tok0, _, tail_logits = eng.tail(0)
    assert np.array_equal(eng.read_logits(0), tail_logits)
    others = list(range(1, ROWS))
    for s in others:
        eng.kv_reset(s, lengths[s])
    _, logits = eng.step_batch(others, [firsts[s] for s in others])
    assert np.array_equal(eng.read_logits(0), tail_logits)
    for i, s in enumerate(others):
        assert np.array_equal(eng.read_logits(s), logits[i]), s


def test_batch16_greedy_steps_track_single_steps(batch16):
    """32 greedy steps (config 4): every 8th step each sequence is re-run
    through the batch-1 path from the same cache state and compared."""
    eng, lengths, _, firsts = batch16
    slots = list(range(ROWS))
    feeds = list(firsts)
    for s in slots:
        eng.kv_reset(s, lengths[s])
    for step in range(STEPS):
        if step % 8 == 0:
            say(f"step {step}")
        greedy, logits = eng.step_batch(slots, feeds)
        for s in slots:
            pos = lengths[s] + step
            assert eng.decode_state(s).token_position == pos + 1
            assert int(greedy[s]) == int(np.argmax(logits[s])), (step, s)
        if step % 8 == 7:
            for s in slots:
                pos = lengths[s] + step
                eng.kv_reset(s, pos)
                tok, _, single = eng.step(s, feeds[s])
                check_logits(int(greedy[s]), logits[s], tok, single, f"step {step} slot {s}")
        feeds = [int(g) for g in greedy]


def test_batch_subsets_order_and_two_groups(batch16):
    """A batch of any slot subset in any order equals stepping each slot of it
    alone; 18 rows run as a group of 16 and a group of 2."""
    eng, lengths, _, firsts = batch16
    extra = {}
    for s in (ROWS, ROWS + 1):
        p = qo.fill_tokens(100 + 37 * (s - ROWS), SEED, PROMPT_STREAM + s, SHAPE.vocab)
        eng.kv_reset(s, 0)
        tok, _, _ = eng.prefill(s, p, want_logits=False)
        extra[s] = (p.size, tok)
    lens = dict(enumerate(lengths)) | {s: n for s, (n, _) in extra.items()}
    feed = dict(enumerate(firsts)) | {s: t for s, (_, t) in extra.items()}
    for order in ([9, 2, 14, 5, 0], [17, 3, 16] + [s for s in range(ROWS) if s != 3]):
        for s in order:
            eng.kv_reset(s, lens[s])
        say(f"batch of {len(order)} slots in scrambled order")
        greedy, logits = eng.step_batch(order, [feed[s] for s in order])
        for i, s in enumerate(order):
            eng.kv_reset(s, lens[s])
            tok, _, single = eng.step(s, feed[s])
            check_logits(int(greedy[i]), logits[i], tok, single, f"{len(order)} rows: slot {s}")


def test_profile_batch_reports_every_kernel(batch16):
    """qd_profile_batch times every batched kernel, reports algorithmic bytes
    and flops per launch, and advances each slot like qd_step_batch."""
    eng, lengths, _, firsts = batch16
    slots = list(range(ROWS))
    for s in slots:
        eng.kv_reset(s, lengths[s])
    say("profile_batch: 2 steps")
    prof = eng.profile_batch(slots, firsts, 2)
    layers = SHAPE.layers
    for name, per_step in (("batch_qkv_kernel", layers), ("batch_attn_kernel", layers),
                           ("batch_oproj_kernel", layers), ("batch_gateup_kernel", layers),
                           ("batch_down_kernel", layers), ("batch_lmhead_kernel", 1),
                           ("batch_argmax_kernel", 1), ("batch_embed_kernel", 1)):
        launches, avg_us, avg_bytes, _ = prof[name]
        assert launches == 2 * per_step, name
        assert avg_us > 0 and avg_bytes > 0, name
    h, inter = SHAPE.hidden, SHAPE.intermediate
    assert prof["batch_gateup_kernel"][3] == 4 * ROWS * inter * h
    assert prof["batch_lmhead_kernel"][3] == 2 * ROWS * SHAPE.vocab * h
    for s in slots:
        assert eng.decode_state(s).token_position == lengths[s] + 2
