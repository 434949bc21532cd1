"""CPU checks of the C-ABI library: it loads, exports every symbol the header
declares, and its host-only paths (status strings, argument validation,
device-less behaviour) work without a GPU."""
import ctypes
import os
import re

import pytest

import qwen_decode as qd

HEADER = os.path.join(os.path.dirname(__file__), "..", "include", "qd", "qwen_decode.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"QD_API\s+[^;(]*?\b(qd_\w+)\s*\(", text, re.S)))


def test_library_exports_every_declared_symbol():
    names = declared_symbols()
    assert len(names) >= 25
    handle = ctypes.CDLL(qd.LIB_PATH)
    missing = [n for n in names if not hasattr(handle, n)]
    assert not missing, missing
    # The Python binding covers the whole ABI too.
    assert set(names) <= set(qd._SIGNATURES), set(names) - set(qd._SIGNATURES)


def test_status_strings_match_lr_status_values():
    # Same numeric values as lr_status_t (include/lrrt/lrrt.h:17-25).
    expected = ["success", "invalid argument", "not initialized", "already initialized",
                "not supported", "runtime error", "device fault"]
    assert [qd.status_string(i) for i in range(7)] == expected
    assert qd.lib().qd_abi_version() == 4


def test_device_count_is_callable():
    assert qd.device_count() >= 0


def test_engine_create_validates_before_touching_a_device():
    with pytest.raises(qd.QdError) as e:
        qd.Engine(heads=14, kv_heads=3)
    assert e.value.status == qd.INVALID_ARGUMENT
    with pytest.raises(qd.QdError) as e:
        qd.Engine(hidden=1024, heads=16)
    assert e.value.status == qd.NOT_SUPPORTED
    # Only the tested attention shape, 14 query heads over 2 KV heads.
    for kv_heads in (7, 14):
        with pytest.raises(qd.QdError) as e:
            qd.Engine(kv_heads=kv_heads)
        assert e.value.status == qd.NOT_SUPPORTED, kv_heads
    with pytest.raises(qd.QdError) as e:
        qd.Engine(capacity=0)
    assert e.value.status == qd.INVALID_ARGUMENT


@pytest.mark.skipif(qd.device_count() > 0, reason="host-without-GPU behaviour")
def test_engine_create_without_gpu_fails_loudly():
    with pytest.raises(qd.QdError) as e:
        qd.Engine(layers=1, vocab=64, capacity=8)
    assert e.value.status == qd.NOT_SUPPORTED
    assert "no HIP device" in str(e.value)
