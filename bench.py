"""Decode benchmark of the Qwen2 FP32 decode path on one GPU. Prints one JSON line.

Workloads (synthetic random-init weights):
  decode   (default) config 2: 24-layer FP32 decoder + tied 151936x896 LM
           head, N(0, 0.02) weights (seed 1), a 512-token uniform random
           prompt, then greedy decode steps with argmax feedback on the device.
           One "step" = one decode token.
  batch16  config 4: 16 independent sequences with contexts uniform in
           [256, 2048] (seed 3) decoded together; one step = one token of
           every sequence (16 tokens).
  long     config 3: config 2's model decoding at KV context 4065..4096.
  prefill  config 5: the 512-token prompt (seed 4) through the MFMA prompt
           path; one step = one prefill of the 512 tokens. The 128 greedy
           decode steps that follow it in config 5 are reported beside it.
  bf16     config 2's model and context with BF16 decoder matrices and an FP32
           tail, on the resident kernel, timed against the FP32 default line's
           engine (interleaved).
  f16      the same with IEEE FP16 decoder matrices.
  layer    config 1: one decoder layer's decode step at KV context 128
           (weights seed 0), cycling over 8 synthetic layers (8 x 59.6 MB,
           more than the 256 MB last-level cache) so every step streams its
           weights from HBM. One "step" = one token through the 8 layers on
           the resident kernel (small-vocabulary tail); value = layer steps/s.
           qd_layer_decode (one layer per call, stream kernels, context
           exactly 128) is timed beside it.

  python bench.py [--workload decode|long|batch16|prefill|bf16|f16|layer] [--steps K]
                  [--warmup W] [--trials T] [--gpus 1] [--no-cpu]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for sub in ("light-rocm-runtime_amd", "oracle"):
    sys.path.insert(0, os.path.join(ROOT, sub))

import numpy as np  # noqa: E402

import qwen_decode as qd  # noqa: E402

METRIC = "decode tokens/s at batch 1 (Qwen2.5-0.5B-shape FP32) + % HBM roofline"
HBM_PEAK_GBS = 8000.0
MFMA_FP32_PEAK_TFLOPS = 157.3
VOCAB = 151936
PROMPT = 512
SEED = 1
PROMPT_STREAM = 0x300000
BATCH_SEED, BATCH_ROWS = 3, 16
LEN_STREAM, BATCH_PROMPT_STREAM = 0x400000, 0x410000
PREFILL_SEED, PREFILL_DECODE = 4, 128

# Algorithmic bytes of one decode token attending over L positions:
# all FP32 weights (24 x 59,649,536 + tied head 544,538,624 + final norm 3,584)
# + K/V reads 24,576 L + new K/V 24,576 + logits 607,744 + embedding row 3,584.
WEIGHT_BYTES = 1_976_131_072


# HBM bytes per decode token of the resident kernels, measured with rocprofv3
# FETCH_SIZE + WRITE_SIZE on the 64-token launch of this workload, scaled by
# the factors a 1 GiB device copy gives in the same profile
# (profiles/roles_kernel_config2.md).
# Re-measured when a kernel changes; None where no measurement exists.
RESIDENT_TRAFFIC_PER_TOKEN = 2_005_670_715
# The role-split kernel on the bench's own 32-token launch of the config-3
# workload (context 4065..4096; profiles/roles_kernel_config3.md).
RESIDENT_TRAFFIC_PER_TOKEN_LONG = 2_102_114_363


def step_bytes(length: int) -> int:
    return WEIGHT_BYTES + 24_576 * length + 24_576 + 607_744 + 3_584


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def stream_tokens(n, seed, stream, vocab):
    """Uniform random tokens from the repository's counter-based generator
    (splitmix64 over a per-(seed, stream) key, the same stream the oracle and
    the tests use), computed here without the oracle."""
    m = (1 << 64) - 1

    def mix(z):
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & m
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & m
        return z ^ (z >> 31)

    key = mix((seed * 0x9E3779B97F4A7C15 + stream * 0xC2B2AE3D27D4EB4F + 0x165667B19E3779F9) & m)
    out = np.empty(n, np.uint32)
    for i in range(n):
        r = mix((key + i * 0x9E3779B97F4A7C15) & m) >> 32
        out[i] = (r * vocab) >> 32
    return out


def roofline_hbm(name, avg_us, avg_bytes, traffic=None):
    achieved = avg_bytes / (avg_us * 1e-6) / 1e9
    return {"bound": "hbm", "kernel": name, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
            "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
            "avg_us": round(avg_us, 3), "bytes_per_launch": round(avg_bytes)}


def dominant(prof):
    """The kernel with the largest total time: (name, (launches, avg_us, avg_bytes, avg_flops))."""
    return max(prof.items(), key=lambda kv: kv[1][0] * kv[1][1])


def mfma_summary(prof, names):
    """Achieved FP32 matrix-core rate over the given kernels' launches."""
    us = sum(prof[n][0] * prof[n][1] for n in names if n in prof)
    fl = sum(prof[n][0] * prof[n][3] for n in names if n in prof)
    tf = fl / (us * 1e-6) / 1e12 if us else 0.0
    return {"kernels": [n for n in names if n in prof], "achieved_tflops": round(tf, 2),
            "peak_tflops": MFMA_FP32_PEAK_TFLOPS, "frac": round(tf / MFMA_FP32_PEAK_TFLOPS, 4)}


# ---- CPU baselines (the oracle, timed on this host's cores) ---------------------

def cpu_decode_baseline(seed, contexts, budget_s=12.0, max_steps=62):
    """The CPU oracle (FP32, OpenMP over host cores, KV cache) timed on decode
    steps of the same model, cycling through `contexts` (synthetic cached KV),
    as many steps as fit the time budget."""
    import qwen_oracle as qo

    model = qo.Model(qo.QWEN25_05B)
    model.fill_synthetic(seed)
    top = max(contexts)
    cache = qo.Cache(model, top + max_steps + 2)
    for layer in range(qo.QWEN25_05B.layers):
        cache.layer(layer, False)[:top] = 0.01
        cache.layer(layer, True)[:top] = 0.01
    cache.decode_step(1, contexts[0], want_logits=False)  # warm caches / threads
    steps, t0 = 0, time.perf_counter()
    while True:
        cache.decode_step(1 + steps, contexts[steps % len(contexts)] + steps // len(contexts),
                          want_logits=False)
        steps += 1
        el = time.perf_counter() - t0
        if el > budget_s or steps >= max_steps:
            break
    model.close()
    return steps, el, qo.threads()


def cpu_prefill_baseline(seed, n):
    import qwen_oracle as qo

    model = qo.Model(qo.QWEN25_05B)
    model.fill_synthetic(seed)
    cache = qo.Cache(model, n + 2)
    prompt = stream_tokens(n, seed, PROMPT_STREAM, VOCAB)
    t0 = time.perf_counter()
    cache.prefill(prompt, want_logits=False)
    el = time.perf_counter() - t0
    model.close()
    return el, qo.threads()


# ---- workloads ------------------------------------------------------------------

CONFIG2_TEXT = ("BASELINE config 2: 24-layer Qwen2.5-0.5B-shape FP32 decoder + tied 151936x896 LM "
                "head, batch 1, prompt 512 then greedy decode with device argmax feedback")
# the same model decoding at KV context up to 4096.
LONG_PROMPT = 4064
CONFIG3_TEXT = ("BASELINE config 3: 24-layer Qwen2.5-0.5B-shape FP32 decoder + tied 151936x896 LM "
                "head, batch 1, prompt 4064 then greedy decode to KV context 4096 with device "
                "argmax feedback")


def run_decode(K, W, no_cpu, trials, with_graph=True):
    return decode_line(K, W, no_cpu, trials, PROMPT, CONFIG2_TEXT, RESIDENT_TRAFFIC_PER_TOKEN, with_graph)


def run_long(K, W, no_cpu, trials, with_graph=True):
    return decode_line(K, W, no_cpu, trials, LONG_PROMPT, CONFIG3_TEXT, RESIDENT_TRAFFIC_PER_TOKEN_LONG,
                       with_graph)


def host_info():
    """The host the CPU baseline ran on: CPU model, logical CPUs, the CPUs this
    process may use, and the OpenMP thread setting."""
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        usable = os.cpu_count()
    return {"cpu_model": model, "nproc": os.cpu_count(), "usable_cpus": usable,
            "omp_num_threads": os.environ.get("OMP_NUM_THREADS")}


def trial_orders(paths):
    """Rotations of the path list, forwards then backwards: trial t runs the
    paths in order t mod 2n (benchmarks/qwen_stateful_graph.cpp:247-261)."""
    n = len(paths)
    orders = [[(off + i) % n for i in range(n)] for off in range(n)]
    orders += [[(off + n - i) % n for i in range(n)] for off in range(n)]
    return [[paths[i] for i in o] for o in orders]


def spread(samples):
    v = sorted(samples)
    mid = len(v) // 2
    med = v[mid] if len(v) % 2 else 0.5 * (v[mid - 1] + v[mid])
    return {"median": med, "min": v[0], "max": v[-1]}


def decode_line(K, W, no_cpu, trials, prompt_len, workload, traffic_per_token, with_graph=True):
    capacity = prompt_len + max(K, W) + 24
    log("engine create + synthetic weights")
    eng = qd.Engine(capacity=capacity, max_batch=1)
    eng.load_synthetic(SEED)
    prompt = stream_tokens(prompt_len, SEED, PROMPT_STREAM, VOCAB)
    log(f"prefill {prompt_len}")
    first, _, _ = eng.prefill(0, prompt, want_logits=False)
    grid = eng.resident_grid()

    # Decode paths over the same K tokens, interleaved over trials:
    # "resident" (qd_generate_resident: one launch, argmax fed back on the
    # device) and the per-token contract of the reference's executor surface
    # (one call per token, its logits copied to the host): "step" (qd_step,
    # one resident-kernel launch per token) and "graph" (qd_step_graph, the
    # stream kernels replayed from the slot's captured HIP graph).
    def resident():
        toks, reason, _ = eng.generate(0, first, K)
        assert len(toks) == K, (len(toks), reason)
        return toks.tolist(), eng.last_timing().total_us

    def step():
        out, tok = [], first
        for _ in range(K):
            tok, _, _ = eng.step(0, tok, want_logits=True)
            out.append(tok)
        return out, None

    def graph():
        out, tok = [], first
        for _ in range(K):
            tok, _, _ = eng.step_graph(0, tok, want_logits=True)
            out.append(tok)
        return out, None

    paths = {"resident": resident, "step": step, "graph": graph}
    if not with_graph:
        del paths["graph"]
    if W:
        log(f"warmup {W} tokens per path")
        eng.generate(0, first, W)
        for fn in (eng.step, eng.step_graph) if with_graph else (eng.step,):
            eng.kv_reset(0, prompt_len)
            tok = first
            for _ in range(W):
                tok = int(fn(0, tok, want_logits=True)[0])
    samples = {name: {"wall_ms": [], "device_us": []} for name in paths}
    tokens = {}
    log(f"timed: {trials} interleaved trials x {K} tokens per path")
    for t in range(trials):
        for name in trial_orders(list(paths))[t % (2 * len(paths))]:
            eng.kv_reset(0, prompt_len)
            eng.sync()
            t0 = time.perf_counter()
            toks, dev_us = paths[name]()
            eng.sync()
            samples[name]["wall_ms"].append((time.perf_counter() - t0) * 1e3)
            if dev_us is not None:
                samples[name]["device_us"].append(dev_us)
            tokens.setdefault(name, toks)
            assert toks == tokens[name], f"{name}: trial {t} produced other tokens"
    # The paths run the same arithmetic: the same greedy chain.
    assert all(tokens[name] == tokens["resident"] for name in paths), \
        "resident, step and graph paths disagree"
    res_wall = spread(samples["resident"]["wall_ms"])
    step_wall = spread(samples["step"]["wall_ms"])
    graph_wall = spread(samples["graph"]["wall_ms"]) if with_graph else None
    total_bytes = sum(step_bytes(prompt_len + 1 + i) for i in range(K))
    tok_s = K / (res_wall["median"] * 1e-3)

    if grid:
        # One resident launch runs all K tokens: its HIP-event duration on the
        # engine stream is the kernel time, its algorithmic bytes the K steps'.
        dev = spread(samples["resident"]["device_us"])
        traffic = traffic_per_token * K if traffic_per_token else None
        roof = roofline_hbm("roles_kernel", dev["median"], float(total_bytes), traffic)
        roof["avg_us_min"] = round(dev["min"], 3)
        roof["avg_us_max"] = round(dev["max"], 3)
    else:
        eng.kv_reset(0, prompt_len)
        prof = eng.profile_kernels(0, first, min(K, 16))
        name, (_, avg_us, avg_bytes, _) = dominant(prof)
        roof = roofline_hbm(name, avg_us, avg_bytes)
    # The step path's kernels, each timed with HIP events.
    eng.kv_reset(0, prompt_len)
    prof = eng.profile_kernels(0, first, min(K, 16))
    log("step-path kernel profile: " + ", ".join(f"{n}={v[1]:.1f}us" for n, v in prof.items()))
    dname, (_, davg_us, davg_bytes, _) = dominant(prof)
    log("HBM probe")
    read_gbs, copy_gbs = qd.probe_hbm(0, 1 << 31, 5)
    eng.close()
    roof["frac_of_measured_read"] = round(roof["achieved"] / read_gbs, 4) if read_gbs else None

    cpu = None
    if not no_cpu:
        steps, el, cores = cpu_decode_baseline(SEED, [prompt_len])
        cpu = {"value": round(steps / el, 3), "unit": "tokens/s", "cores": cores, "kind": "port",
               "sample": f"{steps} decode steps at context {prompt_len + 1}..{prompt_len + steps}, "
                         f"24 layers + 151936-row LM head, oracle/libqwen_oracle.so FP32 OpenMP "
                         f"({cores} threads)",
               "host": host_info()}
    return {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tokens/s",
        "ms_per_step": round(res_wall["median"] / K, 4),
        "higher_is_better": True,
        "dtype": "f32",
        "data": "synthetic: random-init N(0,0.02) weights / N(0,0.01) biases, seed 1; "
                f"{prompt_len} uniform random prompt tokens",
        "config": {
            "workload": workload,
            "batch": 1, "context": f"{prompt_len + 1}..{prompt_len + K}", "layers": 24,
            "hidden": 896, "vocab": VOCAB,
        },
        "trials": {"count": trials, "order": "interleaved rotations, forwards then backwards",
                   "resident_ms": {k: round(v, 3) for k, v in res_wall.items()},
                   "step_ms": {k: round(v, 3) for k, v in step_wall.items()},
                   "graph_ms": {k: round(v, 3) for k, v in graph_wall.items()} if graph_wall else None},
        "step_hbm": {"achieved_gbs": round(total_bytes / (res_wall["median"] * 1e-3) / 1e9, 1),
                     "peak_gbs": HBM_PEAK_GBS, "bytes_per_token": round(total_bytes / K)},
        "device_tokens_per_s": round(K / (roof["avg_us"] * 1e-6), 2) if grid else None,
        "roofline": roof,
        "hbm_measured": {"read_gbs": round(read_gbs, 1), "copy_gbs": round(copy_gbs, 1),
                         "probe": "qd_probe_hbm: best of 5 passes over 2 GiB"},
        # The per-token contract (one call per token, its 607,744-byte
        # logits row copied to the host): qd_step, and the stream kernels
        # replayed from a HIP graph beside it.
        "executor_surface": {
            "path": "qd_step per token: one cooperative launch of the resident kernel + the logits "
                    "copy to the host",
            "tokens_per_s": round(K / (step_wall["median"] * 1e-3), 2),
            "ms_per_token": round(step_wall["median"] / K, 4),
            "graph": {"path": "qd_step_graph per token: the stream-ordered step kernels replayed from "
                              "the slot's captured HIP graph + the logits copy",
                      "tokens_per_s": round(K / (graph_wall["median"] * 1e-3), 2),
                      "ms_per_token": round(graph_wall["median"] / K, 4),
                      "dominant_kernel": roofline_hbm(dname, davg_us, davg_bytes)} if graph_wall else None,
        },
        "cpu_baseline": cpu,
        "path": f"resident megakernel, {grid} workgroups" if grid else "stream-ordered kernels",
    }


# Half-width decoder matrices (BF16 or FP16): the 24 layers' wqkv, wo, gate,
# up and down at 2 bytes per element, their biases and norms, the FP32 tail
# (tied LM head, final norm) as in WEIGHT_BYTES.
HALF_WEIGHT_BYTES = (24 * (2 * (1152 * 896 + 896 * 896 + 3 * 4864 * 896) + 4 * (1152 + 2 * 896))
                     + 544_538_624 + 3_584)
HALF_NAMES = {"bf16": "BF16", "f16": "FP16"}


def run_half(dtype, K, W, no_cpu, trials):
    """Config 2's decode with BF16 or FP16 decoder weights and an FP32 tail
    (the reference's reduced-precision modes, examples/qwen/README.md:291-300),
    on the resident kernel, interleaved with the FP32 default line's engine."""
    label = HALF_NAMES[dtype]
    capacity = PROMPT + max(K, W) + 24
    log(f"engines: {label} decoder weights and FP32, both on the resident kernel")
    engines = {dtype: qd.Engine(capacity=capacity, max_batch=1, decoder_dtype=dtype),
               "f32": qd.Engine(capacity=capacity, max_batch=1)}
    prompt = stream_tokens(PROMPT, SEED, PROMPT_STREAM, VOCAB)
    firsts = {}
    for name, eng in engines.items():
        eng.load_synthetic(SEED)
        log(f"{name}: prefill {PROMPT}")
        firsts[name], _, _ = eng.prefill(0, prompt, want_logits=False)
        if W:
            eng.generate(0, firsts[name], W)
    samples = {name: {"wall_ms": [], "device_us": []} for name in engines}
    log(f"timed: {trials} interleaved trials x {K} tokens per engine")
    for t in range(trials):
        for name in trial_orders(list(engines))[t % 4]:
            eng = engines[name]
            eng.kv_reset(0, PROMPT)
            eng.sync()
            t0 = time.perf_counter()
            toks, _, _ = eng.generate(0, firsts[name], K)
            eng.sync()
            samples[name]["wall_ms"].append((time.perf_counter() - t0) * 1e3)
            samples[name]["device_us"].append(eng.last_timing().total_us)
            assert len(toks) == K
    grid = engines[dtype].resident_grid()
    wh, w32 = spread(samples[dtype]["wall_ms"]), spread(samples["f32"]["wall_ms"])
    dev = spread(samples[dtype]["device_us"])
    for eng in engines.values():
        eng.close()
    per_token = [HALF_WEIGHT_BYTES + 24_576 * (PROMPT + 1 + i) + 24_576 + 607_744 + 3_584 for i in range(K)]
    total = float(sum(per_token))
    roof = roofline_hbm("roles_kernel", dev["median"], total)
    return {
        "metric": f"decode tokens/s at batch 1 (Qwen2.5-0.5B shape, {label} decoder weights + FP32 tail) "
                  "+ % HBM roofline",
        "value": round(K / (wh["median"] * 1e-3), 2),
        "unit": "tokens/s",
        "ms_per_step": round(wh["median"] / K, 4),
        "higher_is_better": True,
        "dtype": "f32",
        "data": f"synthetic: random-init N(0,0.02) weights rounded to {label} for the decoder matrices, "
                f"N(0,0.01) biases, seed 1; {PROMPT} uniform random prompt tokens",
        "config": {
            "workload": f"BASELINE config 2's model and context with {label} decoder matrices (FP32 "
                        "compute, FP32 biases, norms, embeddings and LM head), resident kernel",
            "batch": 1, "context": f"{PROMPT + 1}..{PROMPT + K}", "layers": 24, "hidden": 896,
            "vocab": VOCAB, "decoder_weights": dtype,
        },
        "trials": {"count": trials, "order": "interleaved rotations, forwards then backwards",
                   f"{dtype}_ms": {k: round(v, 3) for k, v in wh.items()},
                   "f32_ms": {k: round(v, 3) for k, v in w32.items()}},
        "step_hbm": {"achieved_gbs": round(total / (wh["median"] * 1e-3) / 1e9, 1),
                     "peak_gbs": HBM_PEAK_GBS, "bytes_per_token": round(total / K)},
        "f32_tokens_per_s": round(K / (w32["median"] * 1e-3), 2),
        "roofline": roof,
        "cpu_baseline": None,
        "path": f"resident megakernel, {grid} workgroups ({label} decoder matrices)",
    }


def run_bf16(K, W, no_cpu, trials):
    return run_half("bf16", K, W, no_cpu, trials)


def run_f16(K, W, no_cpu, trials):
    return run_half("f16", K, W, no_cpu, trials)


def batch_lengths():
    return [256 + int(x) for x in stream_tokens(BATCH_ROWS, BATCH_SEED, LEN_STREAM, 2048 - 256 + 1)]


def run_batch16(K, W, no_cpu, trials):
    lengths = batch_lengths()
    slots = list(range(BATCH_ROWS))
    log("engine create + synthetic weights (seed 3, 16 slots)")
    eng = qd.Engine(capacity=max(lengths) + max(K, W) + 16, max_batch=BATCH_ROWS)
    eng.load_synthetic(BATCH_SEED)
    firsts = []
    log("prefill 16 ragged prompts")
    for s, n in enumerate(lengths):
        eng.kv_reset(s, 0)
        t, _, _ = eng.prefill(s, stream_tokens(n, BATCH_SEED, BATCH_PROMPT_STREAM + s, VOCAB),
                              want_logits=False)
        firsts.append(t)

    def run(steps):
        feeds = list(firsts)
        for _ in range(steps):
            g, _ = eng.step_batch(slots, feeds, want_logits=False)
            feeds = [int(x) for x in g]

    if W:
        log(f"warmup {W}")
        run(W)
    for s in slots:
        eng.kv_reset(s, lengths[s])
    log(f"timed {K} batched steps")
    eng.sync()
    t0 = time.perf_counter()
    run(K)
    eng.sync()
    wall = time.perf_counter() - t0
    for s in slots:
        eng.kv_reset(s, lengths[s])
    prof = eng.profile_batch(slots, firsts, min(K, 8))
    eng.close()
    log("kernel profile: " + ", ".join(f"{n}={v[1]:.1f}us" for n, v in prof.items()))
    name, (_, avg_us, avg_bytes, _) = dominant(prof)
    # Algorithmic bytes of the K steps: weights once per step, every
    # sequence's K/V rows, its new K/V row, logits and embedding row.
    total_bytes = sum(WEIGHT_BYTES + sum(24_576 * (n + 1 + i) + 24_576 + 607_744 + 3_584
                                         for n in lengths) for i in range(K))
    step_gbs = total_bytes / wall / 1e9
    cpu = None
    if not no_cpu:
        steps, el, cores = cpu_decode_baseline(BATCH_SEED, lengths, max_steps=32)
        cpu = {"value": round(steps / el, 3), "unit": "tokens/s", "cores": cores, "kind": "port",
               "sample": f"{steps} single-sequence decode steps cycling over the 16 contexts "
                         f"(synthetic cached KV), oracle/libqwen_oracle.so FP32 OpenMP"}
    gemms = ["batch_qkv_kernel", "batch_oproj_kernel", "batch_gateup_kernel",
             "batch_down_kernel", "batch_lmhead_kernel"]
    return {
        "metric": "batched decode tokens/s (16 ragged sequences, Qwen2.5-0.5B-shape FP32) "
                  "+ % HBM roofline",
        "value": round(BATCH_ROWS * K / wall, 2),
        "unit": "tokens/s",
        "ms_per_step": round(wall * 1e3 / K, 4),
        "higher_is_better": True,
        "dtype": "f32",
        "data": "synthetic: random-init N(0,0.02) weights / N(0,0.01) biases, seed 3; "
                "16 uniform random prompts of uniform [256, 2048] lengths",
        "config": {
            "workload": "BASELINE config 4: 24-layer FP32 model, 16 sequences with ragged "
                        "contexts decoded together (M=16 skinny GEMMs on FP32 MFMA), greedy "
                        "feedback",
            "batch": BATCH_ROWS, "contexts": lengths, "layers": 24, "hidden": 896, "vocab": VOCAB,
        },
        "step_hbm": {"achieved_gbs": round(step_gbs, 1), "peak_gbs": HBM_PEAK_GBS,
                     "frac": round(step_gbs / HBM_PEAK_GBS, 4),
                     "bytes_per_step": round(total_bytes / K)},
        "roofline": roofline_hbm(name, avg_us, avg_bytes),
        "mfma": mfma_summary(prof, gemms),
        "kernels_us": {n: round(v[1], 2) for n, v in prof.items()},
        "cpu_baseline": cpu,
        "path": "stream-ordered batched kernels",
    }


# one decoder layer, one decode step at KV context 128.
LAYER_COPIES = 8          # layers cycled per token: 8 x 59.6 MB > the 256 MB MALL
LAYER_CONTEXT = 128
LAYER_SEED = 0
LAYER_VOCAB = 1024        # the resident launch's tail over a small vocabulary
# Algorithmic bytes of one layer step attending over L positions: the
# layer's FP32 weights, biases and norms + its K/V reads (1,024 L).
LAYER_WEIGHT_BYTES = 59_649_536


def layer_step_bytes(length: int) -> int:
    return LAYER_WEIGHT_BYTES + 1024 * length


def cpu_layer_baseline(budget_s=10.0, max_steps=20000):
    """The CPU oracle's single layer step (FP32, OpenMP) at position 128,
    cycling over LAYER_COPIES layers of the seed-0 model as the GPU line does
    (so the weights stream from DRAM rather than sit in the host's caches),
    as many steps as fit the budget."""
    import qwen_oracle as qo

    model = qo.Model(qo.ModelShape(layers=LAYER_COPIES, vocab=LAYER_VOCAB))
    model.fill_synthetic(LAYER_SEED)
    cache = qo.Cache(model, LAYER_CONTEXT + 2)
    for layer in range(LAYER_COPIES):
        cache.layer(layer, False)[:LAYER_CONTEXT] = 0.01
        cache.layer(layer, True)[:LAYER_CONTEXT] = 0.01
    hidden = np.full(896, 0.01, np.float32)
    for layer in range(LAYER_COPIES):  # warm threads
        cache.layer_step(layer, hidden, LAYER_CONTEXT)
    steps, t0 = 0, time.perf_counter()
    while True:
        cache.layer_step(steps % LAYER_COPIES, hidden, LAYER_CONTEXT)
        steps += 1
        el = time.perf_counter() - t0
        if el > budget_s or steps >= max_steps:
            break
    model.close()
    return steps, el, qo.threads()


def run_layer(K, W, no_cpu, trials):
    log(f"engine create: {LAYER_COPIES} synthetic layers (seed {LAYER_SEED}), vocab {LAYER_VOCAB}")
    eng = qd.Engine(layers=LAYER_COPIES, vocab=LAYER_VOCAB, capacity=LAYER_CONTEXT + max(K, W) + 8,
                    max_batch=1)
    eng.load_synthetic(LAYER_SEED)
    grid = eng.resident_grid()
    first = 1

    # "resident": K tokens in one launch, each through the 8 layers
    # (contexts 129 .. 128 + K), timed by HIP events on the engine stream.
    def resident():
        eng.kv_reset(0, LAYER_CONTEXT)
        toks, reason, _ = eng.generate(0, first, K)
        assert len(toks) == K, (len(toks), reason)
        return eng.last_timing().total_us

    # "layer": qd_layer_decode, one layer per call at context exactly 128
    # (the query at position 128), cycling over the layers.
    def layer_calls():
        eng.sync()
        t0 = time.perf_counter()
        for i in range(K * LAYER_COPIES):
            eng.layer_decode(0, i % LAYER_COPIES, 1, LAYER_CONTEXT + 1)
        eng.sync()
        return (time.perf_counter() - t0) * 1e6

    if W:
        log(f"warmup {W} tokens per path")
        eng.kv_reset(0, LAYER_CONTEXT)
        eng.generate(0, first, W)
        for i in range(W * LAYER_COPIES):
            eng.layer_decode(0, i % LAYER_COPIES, 1, LAYER_CONTEXT + 1)
    samples = {"resident": [], "layer": []}
    paths = {"resident": resident, "layer": layer_calls}
    log(f"timed: {trials} interleaved trials x {K} tokens x {LAYER_COPIES} layers per path")
    for t in range(trials):
        for name in trial_orders(list(paths))[t % 4]:
            samples[name].append(paths[name]())
    eng.close()
    steps = K * LAYER_COPIES
    res_us = spread(samples["resident"])
    lay_us = spread(samples["layer"])
    res_step_us = res_us["median"] / steps
    lay_step_us = lay_us["median"] / steps
    # Bytes of the resident launch's layer steps (the small tail excluded:
    # the figure is a floor on what the layers alone achieve).
    res_bytes = LAYER_COPIES * sum(layer_step_bytes(LAYER_CONTEXT + 1 + i) for i in range(K))
    roof = roofline_hbm("roles_kernel", res_us["median"], float(res_bytes))
    roof["per"] = f"one launch: {K} tokens x {LAYER_COPIES} layer steps"
    lay_gbs = layer_step_bytes(LAYER_CONTEXT + 1) / (lay_step_us * 1e-6) / 1e9
    cpu = None
    if not no_cpu:
        n, el, cores = cpu_layer_baseline()
        cpu = {"value": round(n / el, 2), "unit": "layer-steps/s", "cores": cores, "kind": "port",
               "sample": f"{n} single-layer steps at position 128 cycling over {LAYER_COPIES} layers "
                         f"(synthetic cached KV), oracle/libqwen_oracle.so FP32 OpenMP"}
    return {
        "metric": "single decoder layer decode steps/s (Qwen2 layer shape FP32, KV context 128) "
                  "+ % HBM roofline",
        "value": round(1e6 / res_step_us, 1),
        "unit": "layer-steps/s",
        "ms_per_step": round(res_us["median"] / K / 1e3, 4),
        "higher_is_better": True,
        "dtype": "f32",
        "data": f"synthetic: random-init N(0,0.02) weights / N(0,0.01) biases, seed {LAYER_SEED}; "
                f"{LAYER_COPIES} distinct layers; zero K/V context",
        "config": {
            "workload": "BASELINE config 1: one Qwen2 decoder layer (hidden 896, 14/2 heads, "
                        "intermediate 4864) decode step at KV context 128, batch 1, cycling over "
                        f"{LAYER_COPIES} weight copies",
            "batch": 1, "context": f"{LAYER_CONTEXT + 1}..{LAYER_CONTEXT + K}", "layers": LAYER_COPIES,
            "hidden": 896, "vocab": LAYER_VOCAB,
        },
        "us_per_layer_step": round(res_step_us, 3),
        "trials": {"count": trials, "resident_us": {k: round(v, 2) for k, v in res_us.items()},
                   "layer_decode_us": {k: round(v, 2) for k, v in lay_us.items()}},
        "roofline": roof,
        "layer_decode": {"path": "qd_layer_decode per layer: stream-ordered kernels, context 128",
                         "us_per_layer_step": round(lay_step_us, 3),
                         "achieved_gbs": round(lay_gbs, 1),
                         "frac": round(lay_gbs / HBM_PEAK_GBS, 4)},
        "cpu_baseline": cpu,
        "path": f"resident megakernel, {grid} workgroups" if grid else "stream-ordered kernels",
    }


def run_prefill(K, W, no_cpu, trials):
    prompt = stream_tokens(PROMPT, PREFILL_SEED, PROMPT_STREAM, VOCAB)
    log("engine create + synthetic weights (seed 4)")
    eng = qd.Engine(capacity=PROMPT + PREFILL_DECODE + 8, max_batch=1)
    eng.load_synthetic(PREFILL_SEED)
    for _ in range(W):
        eng.kv_reset(0, 0)
        eng.prefill(0, prompt, want_logits=False)
    log(f"timed {K} prefills of {PROMPT} tokens")
    eng.sync()
    t0 = time.perf_counter()
    for _ in range(K):
        eng.kv_reset(0, 0)
        first, _, _ = eng.prefill(0, prompt, want_logits=False)
    eng.sync()
    wall = time.perf_counter() - t0
    # Config 5's decode phase: 128 greedy steps reusing the prompt's cache.
    eng.sync()
    t1 = time.perf_counter()
    toks, _, _ = eng.generate(0, first, PREFILL_DECODE)
    eng.sync()
    dec_wall = time.perf_counter() - t1
    eng.kv_reset(0, 0)
    prof = eng.profile_prefill(0, prompt)
    eng.close()
    log("kernel profile: " + ", ".join(f"{n}={v[1]:.1f}us" for n, v in prof.items()))
    gemms = [n for n in prof if n.startswith("gemm_nt_kernel")]
    mf = mfma_summary(prof, gemms)
    g_us = sum(prof[n][0] * prof[n][1] for n in gemms)
    g_fl = sum(prof[n][0] * prof[n][3] for n in gemms)
    flops = sum(v[0] * v[3] for v in prof.values())
    cpu = None
    if not no_cpu:
        el, cores = cpu_prefill_baseline(PREFILL_SEED, 256)
        cpu = {"value": round(256 / el, 3), "unit": "tokens/s", "cores": cores, "kind": "port",
               "sample": "one 256-token prefill (same model and prompt stream), "
                         "oracle/libqwen_oracle.so FP32 OpenMP"}
    return {
        "metric": "prefill tokens/s (512-token prompt, Qwen2.5-0.5B-shape FP32) "
                  "+ % FP32 MFMA roofline",
        "value": round(PROMPT * K / wall, 2),
        "unit": "tokens/s",
        "ms_per_step": round(wall * 1e3 / K, 4),
        "higher_is_better": True,
        "dtype": "f32",
        "data": "synthetic: random-init N(0,0.02) weights / N(0,0.01) biases, seed 4; "
                "512 uniform random prompt tokens",
        "config": {
            "workload": "BASELINE config 5: 512-token prefill (dense M=512 GEMMs on FP32 MFMA + "
                        "causal GQA attention), then 128 greedy decode steps",
            "prompt": PROMPT, "layers": 24, "hidden": 896, "vocab": VOCAB,
        },
        "roofline": {"bound": "mfma", "kernel": "gemm_nt_kernel (all projections)",
                     "achieved": round(g_fl / (g_us * 1e-6) / 1e12, 2),
                     "peak": MFMA_FP32_PEAK_TFLOPS, "unit": "TFLOP/s",
                     "frac": mf["frac"], "traffic": None,
                     "avg_us": round(g_us / sum(prof[n][0] for n in gemms), 3),
                     "flops_per_prefill": round(g_fl)},
        "prefill_flops": round(flops),
        "kernels_us": {n: round(v[1], 2) for n, v in prof.items()},
        "decode_after_prefill": {"steps": len(toks),
                                 "tokens_per_s": round(len(toks) / dec_wall, 2)},
        "cpu_baseline": cpu,
        "path": "MFMA prompt path",
    }


def copy_probe(mib: int):
    """Copies `mib` MiB device-to-device through the HIP runtime: a plain copy
    kernel of known size whose FETCH_SIZE / WRITE_SIZE counters calibrate the
    per-dispatch HBM traffic of the decode kernel in the same profile."""
    import ctypes as C

    hip = C.CDLL("libamdhip64.so")
    n = mib << 20
    src, dst = C.c_void_p(), C.c_void_p()
    for p in (src, dst):
        if hip.hipMalloc(C.byref(p), C.c_size_t(n)) != 0:
            raise RuntimeError("hipMalloc failed")
    hip.hipMemset(src, 1, C.c_size_t(n))
    for _ in range(3):
        hip.hipMemcpy(dst, src, C.c_size_t(n), 3)  # device to device
    hip.hipDeviceSynchronize()
    hip.hipFree(src)
    hip.hipFree(dst)
    log(f"copy probe: 3 x {mib} MiB device-to-device")


DEFAULTS = {"decode": (64, 8), "long": (32, 4), "batch16": (32, 4), "prefill": (20, 3), "bf16": (64, 8),
            "f16": (64, 8), "layer": (16, 4)}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--workload", choices=sorted(DEFAULTS), default="decode")
    ap.add_argument("--steps", type=int, default=None)
    ap.add_argument("--warmup", type=int, default=None)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--trials", type=int, default=7,
                    help="interleaved timed trials of K steps (decode workloads); value is the median")
    ap.add_argument("--no-graph", action="store_true",
                    help="decode workloads: leave out the qd_step_graph path (under rocprofv3's kernel "
                         "trace the host faulted inside hipGraphLaunch)")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="also run a plain device copy of MIB MiB (PMC calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for {args.gpus}); the decode path "
              "has no multi-GPU mode in this build", file=sys.stderr)
        sys.exit(2)
    K = args.steps if args.steps is not None else DEFAULTS[args.workload][0]
    W = args.warmup if args.warmup is not None else DEFAULTS[args.workload][1]
    if K <= 0:
        sys.exit("--steps must be positive")
    run = {"decode": run_decode, "long": run_long, "batch16": run_batch16,
           "prefill": run_prefill, "bf16": run_bf16, "f16": run_f16, "layer": run_layer}[args.workload]
    if args.workload in ("decode", "long"):
        out = run(K, W, args.no_cpu, max(1, args.trials), not args.no_graph)
    else:
        out = run(K, W, args.no_cpu, max(1, args.trials))
    if args.copy_probe:
        copy_probe(args.copy_probe)
    line = {"metric": out.pop("metric"), "value": out.pop("value"), "unit": out.pop("unit"),
            "n_gpus": 1, "steps": K, "warmup": W, "ms_per_step": out.pop("ms_per_step"),
            "higher_is_better": out.pop("higher_is_better"), "scaling": "weak",
            "vs_baseline": None}
    line.update(out)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
