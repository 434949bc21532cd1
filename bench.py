"""Decode benchmark: batch-1 FP32 Qwen2.5-0.5B-shape greedy decode on one GPU.

Workload: 24-layer FP32 decoder + tied
151936x896 LM head, random-init N(0, 0.02) weights (seed 1), a 512-token
uniform random prompt, then greedy decode steps with argmax feedback on the
device. One "step" = one decode token. Prints one JSON line.

  python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu]
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
PROMPT = 512
SEED = 1
PROMPT_STREAM = 0x300000

# Algorithmic bytes of one decode token attending over L positions:
# all FP32 weights (24 x 59,649,536 + tied head 544,538,624 + final norm 3,584)
# + K/V reads 24,576 L + new K/V 24,576 + logits 607,744 + embedding row 3,584.
WEIGHT_BYTES = 1_976_131_072


# HBM bytes per decode token of the resident kernel, measured with rocprofv3
# FETCH_SIZE (x2.000) + WRITE_SIZE (x1.000) on the 64-token launch of this
# workload; the factors come from a 1 GiB device copy in the same profile
# (profiles/resident_decode_kernel_config2.md). Re-measured when the kernel
# changes; None where no measurement exists.
RESIDENT_TRAFFIC_PER_TOKEN = 2_024_293_558


def step_bytes(length: int) -> int:
    return WEIGHT_BYTES + 24_576 * length + 24_576 + 607_744 + 3_584


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_baseline(budget_s: float = 12.0):
    """The CPU oracle (FP32, OpenMP over host cores, KV cache) timed on decode
    steps of the same model at the same context length (512 cached positions
    of synthetic KV), as many steps as fit the time budget."""
    import qwen_oracle as qo

    model = qo.Model(qo.QWEN25_05B)
    model.fill_synthetic(SEED)
    cache = qo.Cache(model, PROMPT + 64)
    for layer in range(qo.QWEN25_05B.layers):
        cache.layer(layer, False)[:PROMPT] = 0.01
        cache.layer(layer, True)[:PROMPT] = 0.01
    cache.decode_step(1, PROMPT, want_logits=False)  # warm caches / threads
    steps, t0 = 0, time.perf_counter()
    while True:
        cache.decode_step(1 + steps, PROMPT + 1 + steps, want_logits=False)
        steps += 1
        el = time.perf_counter() - t0
        if el > budget_s or steps >= 62:
            break
    model.close()
    return {"value": round(steps / el, 3), "unit": "tokens/s", "cores": qo.threads(),
            "kind": "port",
            "sample": f"{steps} decode steps at context {PROMPT + 1}..{PROMPT + steps}, "
                      f"24 layers + 151936-row LM head, oracle/libqwen_oracle.so FP32 OpenMP"}


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


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=64)
    ap.add_argument("--warmup", type=int, default=8)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="also run a plain device copy of MIB MiB (PMC calibration)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for {args.gpus}); the decode path "
              "has no multi-GPU mode in this build", file=sys.stderr)
        sys.exit(2)
    K, W = args.steps, args.warmup
    capacity = PROMPT + max(K, W) + 8

    log("engine create + synthetic weights")
    eng = qd.Engine(capacity=capacity, max_batch=1)
    eng.load_synthetic(SEED)
    prompt = qo_tokens(PROMPT)
    log("prefill 512")
    first, _, _ = eng.prefill(0, prompt, want_logits=False)

    if W:
        log(f"warmup {W}")
        eng.generate(0, first, W)
        eng.kv_reset(0, PROMPT)

    log(f"timed {K} decode steps")
    eng.sync()
    t0 = time.perf_counter()
    toks, reason, _ = eng.generate(0, first, K)
    eng.sync()
    wall = time.perf_counter() - t0
    timing = eng.last_timing()
    assert len(toks) == K, (len(toks), reason)
    dev_s = timing.total_us * 1e-6
    tok_s = K / wall
    total_bytes = sum(step_bytes(PROMPT + 1 + i) for i in range(K))
    step_gbs = total_bytes / dev_s / 1e9

    grid = eng.resident_grid()
    if grid:
        # One resident launch runs all K tokens: its HIP-event duration on the
        # engine stream is the kernel time, its algorithmic bytes the K steps'.
        dom_name, avg_us, avg_bytes = "resident_decode_kernel", timing.total_us, float(total_bytes)
        traffic = RESIDENT_TRAFFIC_PER_TOKEN * K if RESIDENT_TRAFFIC_PER_TOKEN else None
    else:
        eng.kv_reset(0, PROMPT)
        prof = eng.profile_kernels(0, first, min(K, 16))
        dom_name, (launches, avg_us, avg_bytes) = max(prof.items(), key=lambda kv: kv[1][0] * kv[1][1])
        traffic = None
        log("kernel profile: " + ", ".join(f"{n}={v[1]:.1f}us" for n, v in prof.items()))
    achieved = avg_bytes / (avg_us * 1e-6) / 1e9
    eng.close()

    if args.copy_probe:
        copy_probe(args.copy_probe)
    cpu = None if args.no_cpu else cpu_baseline()
    out = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": K,
        "warmup": W,
        "ms_per_step": round(wall * 1e3 / K, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic: random-init N(0,0.02) weights / N(0,0.01) biases, seed 1; "
                "512 uniform random prompt tokens",
        "config": {
            "workload": "BASELINE config 2: 24-layer Qwen2.5-0.5B-shape FP32 decoder + tied "
                        "151936x896 LM head, batch 1, prompt 512 then greedy decode with "
                        "device argmax feedback",
            "batch": 1, "context": f"{PROMPT + 1}..{PROMPT + K}", "layers": 24,
            "hidden": 896, "vocab": 151936,
        },
        "step_hbm": {"achieved_gbs": round(step_gbs, 1), "peak_gbs": HBM_PEAK_GBS,
                     "frac": round(step_gbs / HBM_PEAK_GBS, 4),
                     "bytes_per_token": round(total_bytes / K)},
        "device_tokens_per_s": round(K / dev_s, 2),
        "roofline": {"bound": "hbm", "kernel": dom_name, "achieved": round(achieved, 1),
                     "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic, "avg_us": round(avg_us, 3),
                     "bytes_per_launch": round(avg_bytes)},
        "cpu_baseline": cpu,
        "path": f"resident megakernel, {grid} workgroups" if grid else "stream-ordered kernels",
    }
    print(json.dumps(out), flush=True)


def qo_tokens(n):
    """Uniform random prompt tokens from the shared generator specification
    (same stream the tests use), computed here without the oracle."""
    m = (1 << 64) - 1

    def mix(z):
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & m
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & m
        return z ^ (z >> 31)

    key = mix((SEED * 0x9E3779B97F4A7C15 + PROMPT_STREAM * 0xC2B2AE3D27D4EB4F + 0x165667B19E3779F9) & m)
    out = np.empty(n, np.uint32)
    for i in range(n):
        r = mix((key + i * 0x9E3779B97F4A7C15) & m) >> 32
        out[i] = (r * 151936) >> 32
    return out


if __name__ == "__main__":
    main()
