"""Pins the CPU oracle before anything is compared against it.

Each check is chosen so that a plausible mistake (dropped term, wrong sign or
index, transposed operand) fails one of them: closed forms, FP64 brute force
on small inputs, special cases, the Hugging Face FP32 fixtures in
tests/golden/, and planted mistakes that must be caught.
"""
import math
import os

import numpy as np
import pytest

import qwen_oracle as qo

GOLDEN = os.path.join(os.path.dirname(__file__), "golden")


# ---- generator ---------------------------------------------------------------

def test_rng_known_answers():
    # splitmix64 finaliser over key = mix(seed*phi + stream*c + k0): the values
    # below pin the specification the engine implements independently.
    def mix(z):
        m = (1 << 64) - 1
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & m
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & m
        return z ^ (z >> 31)

    m = (1 << 64) - 1
    for seed, stream, counter in [(0, 0, 0), (1, 0x102, 7), (3, 0x7fff00, 123456789), (2**63, 5, 2**40)]:
        key = mix((seed * 0x9E3779B97F4A7C15 + stream * 0xC2B2AE3D27D4EB4F + 0x165667B19E3779F9) & m)
        want = mix((key + counter * 0x9E3779B97F4A7C15) & m)
        assert qo.rng_u64(seed, stream, counter) == want


def test_rng_normal_moments_and_box_muller():
    x = qo.fill_normal(1 << 20, seed=5, stream=9).astype(np.float64)
    assert abs(x.mean()) < 5e-3
    assert abs(x.std() - 1.0) < 5e-3
    # Fourth moment of a normal is 3; a uniform or a halved variance would miss.
    assert abs((x**4).mean() - 3.0) < 0.05
    # Box-Muller from the raw words, for a few indices.
    for i in (0, 1, 99):
        a, b = qo.rng_u64(5, 9, 2 * i), qo.rng_u64(5, 9, 2 * i + 1)
        u1 = ((a >> 11) + 1) * 2.0**-53
        u2 = (b >> 11) * 2.0**-53
        assert x[i] == np.float32(math.sqrt(-2 * math.log(u1)) * math.cos(2 * math.pi * u2))


def test_rng_tokens_uniform_in_range():
    t = qo.fill_tokens(200000, seed=1, stream=0x300000, vocab=151936)
    assert t.max() < 151936
    counts = np.bincount((t * 16 // 151936).astype(np.int64), minlength=16)
    assert counts.min() > 0.9 * 200000 / 16


def test_bench_prompt_stream_is_the_oracles():
    """bench.py draws its prompts with its own copy of the token generator;
    the GPU tests that replay a bench workload draw them from the oracle."""
    import importlib.util
    spec = importlib.util.spec_from_file_location(
        "bench_mod", os.path.join(os.path.dirname(__file__), "..", "bench.py"))
    bench = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(bench)
    for n, seed, stream in ((512, 1, 0x300000), (64, 3, 0x410005), (512, 4, 0x300000)):
        assert np.array_equal(bench.stream_tokens(n, seed, stream, 151936),
                              qo.fill_tokens(n, seed, stream, 151936)), (n, seed, stream)


def test_synthetic_fill_distributions():
    shape = qo.ModelShape(hidden=128, heads=2, kv_heads=1, head_dim=64, intermediate=256, vocab=300, layers=2)
    m = qo.Model(shape)
    m.fill_synthetic(seed=3)
    assert np.all(m.tensor(1, qo.ATTN_NORM) == 1.0)
    assert np.all(m.tensor(0, qo.FINAL_NORM) == 1.0)
    assert abs(m.tensor(0, qo.GATE_W).std() - 0.02) < 1e-3
    assert abs(m.tensor(1, qo.Q_B).std() - 0.01) < 3e-3
    # Distinct streams per layer and tensor.
    assert not np.array_equal(m.tensor(0, qo.UP_W), m.tensor(1, qo.UP_W))
    assert not np.array_equal(m.tensor(0, qo.UP_W), m.tensor(0, qo.GATE_W))
    # Tied head aliases the embedding storage.
    assert np.shares_memory(m.tensor(0, qo.EMBED), m.tensor(0, qo.LM_HEAD))
    expect = qo.fill_normal(shape.vocab * shape.hidden, 3, qo.tail_stream(0), 0.0, 0.02)
    assert np.array_equal(m.tensor(0, qo.EMBED), expect)


# ---- primitives ----------------------------------------------------------------

@pytest.mark.parametrize("c", [0.5, -3.0, 1e-3, 40.0])
def test_rmsnorm_constant_vector_closed_form(c):
    n = 896
    w = (1.0 + 0.001 * np.arange(n)).astype(np.float32)
    x = np.full(n, c, np.float32)
    out = qo.rmsnorm(x, w, 1e-6)
    want = c / math.sqrt(c * c + 1e-6) * w.astype(np.float64)
    np.testing.assert_allclose(out, want, rtol=2e-7)


def test_rmsnorm_eps_matters():
    x = np.full(8, 1e-3, np.float32)
    w = np.ones(8, np.float32)
    out = qo.rmsnorm(x, w, 1e-6)
    np.testing.assert_allclose(out, 1e-3 / math.sqrt(1e-6 + 1e-6), rtol=1e-6)


def test_gemv_dyadic_exact_and_bias():
    rng = np.random.default_rng(0)
    w = (rng.integers(-64, 64, (37, 896)) / 64.0).astype(np.float32)
    x = (rng.integers(-64, 64, 896) / 32.0).astype(np.float32)
    b = (rng.integers(-8, 8, 37) / 4.0).astype(np.float32)
    y = qo.gemv(w, x, b)
    want = w.astype(np.float64) @ x.astype(np.float64) + b
    assert np.array_equal(y, want.astype(np.float32))
    # Transposed-operand mistake would change a non-square product.
    assert not np.allclose(qo.gemv(w, x), (w.astype(np.float64) @ x) + 1.0)


def test_gemv_random_fp64_brute_force():
    rng = np.random.default_rng(1)
    w = rng.standard_normal((64, 4864)).astype(np.float32)
    x = rng.standard_normal(4864).astype(np.float32)
    want = (w.astype(np.float64) @ x.astype(np.float64)).astype(np.float32)
    np.testing.assert_array_equal(qo.gemv(w, x), want)


def test_rope_position_zero_is_identity():
    cos, sin = qo.rope_tables(1e6, 64, 8)
    assert np.all(cos[0] == 1.0) and np.all(sin[0] == 0.0)
    v = np.random.default_rng(2).standard_normal(14 * 64).astype(np.float32)
    assert np.array_equal(qo.rope_apply(v, 64, cos[0], sin[0]), v)


def test_rope_unit_vector_rotation():
    p = 100
    cos, sin = qo.rope_tables(1e6, 64, p + 1)
    for i in (0, 5, 31):
        v = np.zeros(64, np.float32)
        v[i] = 1.0  # (a, b) = (1, 0) -> (cos, sin)
        out = qo.rope_apply(v, 64, cos[p], sin[p])
        angle = p * 1e6 ** (-2 * i / 64)
        assert abs(out[i] - math.cos(angle)) < 2e-6
        assert abs(out[i + 32] - math.sin(angle)) < 2e-6
        w = np.zeros(64, np.float32)
        w[i + 32] = 1.0  # (a, b) = (0, 1) -> (-sin, cos)
        out = qo.rope_apply(w, 64, cos[p], sin[p])
        assert abs(out[i] + math.sin(angle)) < 2e-6
        assert abs(out[i + 32] - math.cos(angle)) < 2e-6


def test_rope_preserves_norm_per_head():
    cos, sin = qo.rope_tables(1e6, 64, 600)
    v = np.random.default_rng(3).standard_normal(16 * 64).astype(np.float32)
    out = qo.rope_apply(v, 64, cos[577], sin[577])
    np.testing.assert_allclose(np.linalg.norm(out.reshape(16, 64), axis=1),
                               np.linalg.norm(v.reshape(16, 64), axis=1), rtol=1e-5)


def test_attention_single_position_returns_v():
    rng = np.random.default_rng(4)
    q = rng.standard_normal(14 * 64).astype(np.float32)
    k = rng.standard_normal((1, 128)).astype(np.float32)
    v = rng.standard_normal((1, 128)).astype(np.float32)
    out = qo.attention(q, k, v, 14, 2, 64).reshape(14, 64)
    for h in range(14):
        assert np.array_equal(out[h], v[0, (h // 7) * 64:(h // 7 + 1) * 64])


def test_attention_equal_keys_give_mean_of_v_and_grouping():
    rng = np.random.default_rng(5)
    L = 9
    q = rng.standard_normal(14 * 64).astype(np.float32)
    k = np.tile(rng.standard_normal(128).astype(np.float32), (L, 1))
    v = rng.standard_normal((L, 128)).astype(np.float32)
    out = qo.attention(q, k, v, 14, 2, 64).reshape(14, 64)
    mean = v.astype(np.float64).mean(axis=0)
    for h in range(14):
        g = h // 7  # heads 0..6 -> KV head 0, 7..13 -> KV head 1
        np.testing.assert_allclose(out[h], mean[g * 64:(g + 1) * 64], rtol=1e-5, atol=1e-6)


def test_attention_fp64_brute_force():
    rng = np.random.default_rng(6)
    L = 33
    q = rng.standard_normal(14 * 64).astype(np.float32)
    k = rng.standard_normal((L, 128)).astype(np.float32)
    v = rng.standard_normal((L, 128)).astype(np.float32)
    out = qo.attention(q, k, v, 14, 2, 64).reshape(14, 64)
    for h in range(14):
        g = h // 7
        s = k[:, g * 64:(g + 1) * 64].astype(np.float64) @ q[h * 64:(h + 1) * 64].astype(np.float64) / 8.0
        p = np.exp(s - s.max())
        want = (p / p.sum()) @ v[:, g * 64:(g + 1) * 64].astype(np.float64)
        np.testing.assert_allclose(out[h], want, rtol=1e-6, atol=1e-7)


def test_silu_mul_closed_forms():
    assert qo.silu_mul(0.0, 5.0) == 0.0
    assert qo.silu_mul(30.0, 2.0) == pytest.approx(60.0, rel=1e-7)
    assert qo.silu_mul(-30.0, 2.0) == pytest.approx(-60.0 * math.exp(-30.0), rel=1e-5)
    g = 1.25
    assert qo.silu_mul(g, 3.0) == pytest.approx(g / (1 + math.exp(-g)) * 3.0, rel=1e-7)


def test_argmax_ties_nan_and_degenerate():
    v = np.array([1.0, 3.0, 2.0, 3.0], np.float32)
    assert qo.argmax(v) == (1, 3.0)
    v = np.array([np.nan, 1.0, np.nan, 1.0], np.float32)
    assert qo.argmax(v)[0] == 1
    assert qo.argmax(np.full(5, -np.inf, np.float32))[0] == 0
    assert qo.argmax(np.full(3, np.nan, np.float32))[0] == 0xFFFFFFFF
    assert qo.argmax(np.zeros(7, np.float32))[0] == 0


# ---- composition against Hugging Face -------------------------------------------

def _load_fixture(name):
    z = np.load(os.path.join(GOLDEN, f"{name}.npz"))
    h, heads, kvh, hd, inter, vocab, layers = (int(x) for x in z["shape"])
    shape = qo.ModelShape(hidden=h, heads=heads, kv_heads=kvh, head_dim=hd, intermediate=inter,
                          vocab=vocab, layers=layers, eps=float(z["eps"]), rope_theta=float(z["rope_theta"]))
    return z, shape


def _run_oracle(z, shape, model):
    prompt = z["prompt"].astype(np.uint32)
    tokens = z["tokens"]
    cache = qo.Cache(model, capacity=len(prompt) + len(tokens) + 1)
    outs = []
    tok, top, logits = cache.prefill(prompt)
    outs.append((tok, logits))
    for i, t in enumerate(tokens[:-1]):
        # Teacher-forced with the Hugging Face token so every step is compared.
        tok, top, logits = cache.decode_step(int(t), len(prompt) + i)
        outs.append((tok, logits))
    return outs


@pytest.mark.parametrize("name", ["hf_tiny", "hf_qwen_layer"])
def test_oracle_matches_hugging_face(name):
    z, shape = _load_fixture(name)
    model = qo.Model(shape)
    model.fill_synthetic(int(z["seed"]))
    outs = _run_oracle(z, shape, model)
    ref = z["logits"]
    for step, (tok, logits) in enumerate(outs):
        rel = np.abs(logits - ref[step]).max() / np.abs(ref[step]).max()
        assert rel < 2e-6, (step, rel)
        assert tok == int(z["tokens"][step])


def test_rope_tables_match_hugging_face():
    z = np.load(os.path.join(GOLDEN, "hf_tiny.npz"))
    pos = z["rope_positions"]
    cos, sin = qo.rope_tables(float(z["rope_theta"]), 64, int(pos.max()) + 1)
    hf_cos, hf_sin = z["rope_cos"], z["rope_sin"]
    # HF duplicates the 32 frequencies across the two halves.
    assert np.array_equal(hf_cos[:, :32], hf_cos[:, 32:])
    # Same FP32 angle; cos/sin agree to an ulp or two of the FP32 result.
    np.testing.assert_allclose(cos[pos], hf_cos[:, :32], rtol=0, atol=4e-7)
    np.testing.assert_allclose(sin[pos], hf_sin[:, :32], rtol=0, atol=4e-7)


@pytest.mark.parametrize("mistake", ["no_qkv_bias", "transposed_o", "swapped_kv_heads", "sign_of_sin"])
def test_planted_mistakes_are_caught(mistake):
    """A plausible mistake planted in the oracle's inputs must break the HF match."""
    z, shape = _load_fixture("hf_tiny")
    model = qo.Model(shape)
    model.fill_synthetic(int(z["seed"]))
    if mistake == "no_qkv_bias":
        for layer in range(shape.layers):
            for kind in (qo.Q_B, qo.K_B, qo.V_B):
                model.tensor(layer, kind)[:] = 0.0
    elif mistake == "transposed_o":
        o = model.tensor(0, qo.O_W).reshape(shape.hidden, shape.heads * shape.head_dim)
        o[:] = o.T.copy()  # square in this shape
    elif mistake == "swapped_kv_heads":
        k = model.tensor(0, qo.K_W).reshape(shape.kv_heads, -1)
        k[:] = k[::-1].copy()
    elif mistake == "sign_of_sin":
        # Conjugate rotation == negated sin: emulate by mirroring the Q/K rows
        # of the second half, which is what a flipped rotate_half sign does to
        # every position except 0.
        for kind, heads in ((qo.Q_W, shape.heads), (qo.K_W, shape.kv_heads)):
            w = model.tensor(0, kind).reshape(heads, 2, shape.head_dim // 2, shape.hidden)
            w[:, 1] *= -1.0
        for kind, heads in ((qo.Q_B, shape.heads), (qo.K_B, shape.kv_heads)):
            b = model.tensor(0, kind).reshape(heads, 2, shape.head_dim // 2)
            b[:, 1] *= -1.0
    outs = _run_oracle(z, shape, model)
    worst = max(np.abs(lg - z["logits"][i]).max() / np.abs(z["logits"][i]).max() for i, (_, lg) in enumerate(outs))
    assert worst > 1e-3, worst
