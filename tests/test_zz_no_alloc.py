"""qd_step_batch_noalloc, the batched step whose scratch is the library's
static device workspace, against qd_step_batch (same kernels, engine-owned
workspace): tokens, logits and K/V rows bit for bit, on two calls in a row,
the second with fewer sequences (the workspace keeps the first call's
contents). After the first call, further calls change neither the device's
free memory (hipMemGetInfo) nor the engine's own allocations."""
import ctypes as C

import numpy as np
import pytest

import qwen_decode as qd
import qwen_oracle as qo

pytestmark = pytest.mark.gpu

GROUP = 16
VOCAB = 4096


def say(msg):
    print(f"[gpu-case] {msg}", flush=True)


def engine_hip_runtime():
    """The HIP runtime library the engine library runs on, by the path mapped
    into this process. torch, when an earlier test imported it, maps a HIP
    runtime of its own under the same name, and that copy does not see the
    engine's device state; so the copy is picked by path, not by name."""
    qd.lib()
    paths = []
    with open("/proc/self/maps") as f:
        for line in f:
            parts = line.split()
            if len(parts) >= 6 and "libamdhip64" in parts[5] and parts[5] not in paths:
                paths.append(parts[5])
    mine = [p for p in paths if "/torch/" not in p]
    return C.CDLL(mine[0] if mine else "libamdhip64.so")


def free_device_bytes():
    """hipMemGetInfo's free bytes of the current device, through the engine's
    HIP runtime."""
    hip = engine_hip_runtime()
    free, total = C.c_size_t(), C.c_size_t()
    assert hip.hipMemGetInfo(C.byref(free), C.byref(total)) == 0
    return int(free.value)


def test_noalloc_batch_step_equals_batch_step():
    say("qd_step_batch_noalloc vs qd_step_batch: 16 then 5 sequences")
    eng = qd.Engine(layers=2, vocab=VOCAB, capacity=64, max_batch=2 * GROUP)
    try:
        eng.load_synthetic(5)
        prompts = [qo.fill_tokens(3 + (i * 7) % 11, 5, 0x300000 + i, VOCAB) for i in range(GROUP)]
        for i, p in enumerate(prompts):
            for slot in (i, GROUP + i):
                eng.kv_reset(slot, 0)
                eng.prefill(slot, p, want_logits=False)
        feeds = np.array([int(p[-1]) for p in prompts], np.uint32)
        a = np.arange(GROUP, dtype=np.uint32)
        g1, l1 = eng.step_batch_noalloc(a, feeds)
        g2, l2 = eng.step_batch(a + GROUP, feeds)
        assert np.array_equal(g1, g2) and np.array_equal(l1, l2)
        for i, p in enumerate(prompts):
            assert eng.decode_state(i).token_position == len(p) + 1
            for layer in (0, 1):
                k1, v1 = eng.read_kv(i, layer, len(p), 1)
                k2, v2 = eng.read_kv(GROUP + i, layer, len(p), 1)
                assert np.array_equal(k1, k2) and np.array_equal(v1, v2), (i, layer)
        # A smaller second call, scrambled slots, greedy tokens fed back; it
        # allocates nothing on the device.
        sel = np.array([3, 0, 11, 7, 14], np.uint32)
        free0, own0 = free_device_bytes(), eng.device_bytes()
        g3, l3 = eng.step_batch_noalloc(sel, g1[sel])
        assert free_device_bytes() == free0 and eng.device_bytes() == own0
        g4, l4 = eng.step_batch(sel + GROUP, g2[sel])
        assert np.array_equal(g3, g4) and np.array_equal(l3, l4)
        for j, i in enumerate(sel.tolist()):
            assert g3[j] == int(np.argmax(l3[j]))
            k1, v1 = eng.read_kv(i, 1, len(prompts[i]) + 1, 1)
            k2, v2 = eng.read_kv(GROUP + i, 1, len(prompts[i]) + 1, 1)
            assert np.array_equal(k1, k2) and np.array_equal(v1, v2), i
        with pytest.raises(qd.QdError) as err:
            eng.step_batch_noalloc(np.arange(GROUP + 1, dtype=np.uint32),
                                   np.zeros(GROUP + 1, np.uint32))
        assert err.value.status == qd.INVALID_ARGUMENT and "1..16" in str(err.value)
    finally:
        eng.close()
