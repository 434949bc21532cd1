"""The prompt path's GEMMs next to the vendor FP32 GEMM at the same shapes.

Times `A . W^T` in FP32 through torch (hipBLASLt / rocBLAS, TF32 off) for the
four projection shapes of a 512-token prompt, and the engine's own prompt
kernels over one prefill (`qd_profile_prefill`: each kernel with its fused
epilogue or split-K reduction). Prints one line per shape. Needs a GPU. The
torch timings run in a child process: torch brings its own HIP runtime, which
does not initialise in a process that already uses the engine's.

    python3 light-rocm-runtime_amd/gemm_reference.py
"""
from __future__ import annotations

import json
import os
import subprocess
import sys

import numpy as np

sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
import qwen_decode as qd  # noqa: E402

ROWS = 512
# (engine kernel name, n, k): the projections of one layer of the prompt path.
SHAPES = (("gemm_nt_kernel:gateup+swiglu", 2 * 4864, 896),
          ("gemm_nt_kernel:down+norm", 896, 4864),
          ("gemm_nt_kernel:qkv+rope", 1152, 896),
          ("gemm_nt_kernel:o+norm", 896, 896))


def vendor_us(m: int, n: int, k: int, reps: int = 20) -> float:
    import torch

    torch.backends.cuda.matmul.allow_tf32 = False
    a = torch.randn(m, k, device="cuda")
    w = torch.randn(n, k, device="cuda")
    for _ in range(3):
        a @ w.t()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        a @ w.t()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) * 1e3 / reps


def main() -> int:
    if len(sys.argv) > 1 and sys.argv[1] == "--vendor":
        print(json.dumps([vendor_us(ROWS, n, k) for _, n, k in SHAPES]))
        return 0
    child = subprocess.run([sys.executable, os.path.abspath(__file__), "--vendor"], check=True,
                           capture_output=True, text=True)
    vendor = json.loads(child.stdout.strip().splitlines()[-1])
    eng = qd.Engine(capacity=ROWS + 8, max_batch=1)
    try:
        eng.load_synthetic(4)
        rng = np.random.default_rng(4)
        prompt = rng.integers(0, eng.config.vocab, ROWS, dtype=np.uint32)
        eng.kv_reset(0, 0)
        prof = eng.profile_prefill(0, prompt)
    finally:
        eng.close()
    print(f"{'kernel':34s} {'shape (m x n x k)':>20s} {'engine us':>10s} {'TFLOP/s':>8s} "
          f"{'vendor us':>10s} {'TFLOP/s':>8s}")
    for (name, n, k), lib in zip(SHAPES, vendor):
        flops = 2.0 * ROWS * n * k
        ours = prof[name][1]
        print(f"{name:34s} {f'{ROWS} x {n} x {k}':>20s} {ours:10.1f} {flops / ours / 1e6:8.1f} "
              f"{lib:10.1f} {flops / lib / 1e6:8.1f}")
    return 0


if __name__ == "__main__":
    sys.exit(main())
