import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("oracle", "light-rocm-runtime_amd"):
    path = os.path.join(ROOT, sub)
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through the C-ABI engine)")
    config.addinivalue_line("markers", "slow: long CPU oracle run")


def pytest_collection_modifyitems(config, items):
    # GPU tests are collected everywhere but only run where a GPU is visible.
    if os.environ.get("QD_FORCE_GPU_TESTS") == "1":
        return
    try:
        import qwen_decode as qd

        has_gpu = qd.device_count() > 0
    except Exception:  # library not built or no HIP runtime
        has_gpu = False
    if has_gpu:
        return
    skip = pytest.mark.skip(reason="no GPU visible")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)
