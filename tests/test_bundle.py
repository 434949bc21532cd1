"""Weight-bundle I/O against the reference's own reader/writer.

oracle/_ref/libref_bundle.so is the reference's header-only
executor/qwen/weight_bundle.hpp compiled from /root/reference (oracle/Makefile);
it only exists in a container that has the reference tree. The known-answer
cases restate tests/qwen_weight_bundle.cpp:157-241 of the reference.
"""
import ctypes as C
import os

import numpy as np
import pytest

import qwen_decode as qd

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF_LIB = os.path.join(ROOT, "oracle", "_ref", "libref_bundle.so")

TENSORS = ["attention_norm_weight", "mlp_norm_weight", "q_weight", "k_weight", "v_weight",
           "q_bias", "k_bias", "v_bias", "out_weight", "gate_weight", "up_weight", "down_weight"]


def counts(shape6):
    keys, h, heads, kvh, hd, inter = shape6
    q, kv = heads * hd, kvh * hd
    return [h, h, q * h, kv * h, kv * h, q, kv, kv, h * q, inter * h, inter * h, h * inter]


def ref_lib():
    if not os.path.exists(REF_LIB):
        pytest.skip("reference bundle checker not built (needs /root/reference)")
    lib = C.CDLL(REF_LIB)
    lib.ref_last_error.restype = C.c_char_p
    lib.ref_load_layer.restype = C.c_longlong
    lib.ref_load_layer.argtypes = [C.c_char_p, C.POINTER(C.c_uint32), C.POINTER(C.c_float),
                                   C.POINTER(C.c_float), C.c_size_t]
    lib.ref_write_layer.argtypes = [C.c_char_p, C.c_char_p, C.POINTER(C.c_uint32), C.c_float,
                                    C.POINTER(C.c_float)]
    lib.ref_load_tail.restype = C.c_longlong
    lib.ref_load_tail.argtypes = [C.c_char_p, C.POINTER(C.c_uint32), C.POINTER(C.c_uint32),
                                  C.POINTER(C.c_uint32), C.c_size_t, C.POINTER(C.c_size_t),
                                  C.POINTER(C.c_float), C.c_size_t]
    lib.ref_write_tail.argtypes = [C.c_char_p, C.c_char_p, C.c_uint32, C.c_uint32,
                                   C.POINTER(C.c_uint32), C.c_size_t, C.POINTER(C.c_float),
                                   C.POINTER(C.c_float), C.POINTER(C.c_float)]
    return lib


def fp(a):
    return a.ctypes.data_as(C.POINTER(C.c_float))


def up(a):
    return a.ctypes.data_as(C.POINTER(C.c_uint32))


def known_answer_data(shape6):
    # tests/qwen_weight_bundle.cpp:52-69,125-133: tensor t holds seed_t + 0.001*i.
    vals = []
    for seed, n in zip(range(1, 13), counts(shape6)):
        vals.append(np.float32(seed) + np.float32(0.001) * np.arange(n, dtype=np.float32))
    return np.concatenate(vals).astype(np.float32)


def manifest_text(shape6, data_file, skip=None, dtype="f32", theta="1000000.0"):
    keys, h, heads, kvh, hd, inter = shape6
    lines, off = [], 0
    for name, n in zip(TENSORS, counts(shape6)):
        if name != skip:
            lines.append(f'    {{"name":"{name}","offset":{off},"count":{n}}}')
        off += 4 * n
    return ("{\n  \"format\": \"lrrt.mini_decoder_weights\",\n  \"version\": 2,\n"
            f"  \"dtype\": \"{dtype}\",\n  \"data\": \"{data_file}\",\n  \"keys\": {keys},\n"
            f"  \"hidden\": {h},\n  \"heads\": {heads},\n  \"kv_heads\": {kvh},\n"
            f"  \"head_dim\": {hd},\n  \"intermediate\": {inter},\n  \"rope_theta\": {theta},\n"
            "  \"tensors\": [\n" + ",\n".join(lines) + "\n  ]\n}\n")


SHAPE = [4, 8, 2, 1, 4, 12]


def test_known_answer_layer_load(tmp_path):
    data = known_answer_data(SHAPE)
    data.tofile(tmp_path / "weights.bin")
    (tmp_path / "weights.json").write_text(manifest_text(SHAPE, "weights.bin"))
    shape, theta, t = qd.bundle_read_layer(str(tmp_path / "weights.json"))
    assert list(shape) == SHAPE and theta == 1e6
    offs = np.cumsum([0] + counts(SHAPE))
    get = lambda i: t[offs[i]:offs[i + 1]]
    # Values asserted by tests/qwen_weight_bundle.cpp:169-183.
    assert abs(get(0)[0] - 1.0) < 1e-5
    assert abs(get(1)[-1] - 2.007) < 1e-5
    assert abs(get(2)[0] - 3.0) < 1e-5
    assert abs(get(5)[0] - 6.0) < 1e-5
    assert abs(get(6)[-1] - 7.003) < 1e-5
    assert abs(get(7)[-1] - 8.003) < 1e-5
    assert abs(get(11)[-1] - 12.095) < 1e-5
    assert np.array_equal(t, data)


@pytest.mark.parametrize("case,needle", [
    ("missing", "missing mini decoder weight tensor: down_weight"),
    ("parent", "invalid mini decoder weight data path"),
    ("dtype", "unsupported mini decoder weight dtype"),
    ("absolute", "invalid mini decoder weight data path"),
    ("short", "mini decoder weight data size mismatch"),
    ("gqa", "invalid GQA shape"),
])
def test_layer_validation_errors(tmp_path, case, needle):
    data = known_answer_data(SHAPE)
    data.tofile(tmp_path / "weights.bin")
    shape = SHAPE
    kw = {}
    name = "weights.bin"
    if case == "missing":
        kw["skip"] = "down_weight"
    elif case == "parent":
        name = "../weights.bin"
    elif case == "dtype":
        kw["dtype"] = "bf16"
    elif case == "absolute":
        name = str(tmp_path / "weights.bin")
    elif case == "short":
        np.concatenate([data, np.zeros(3, np.float32)]).tofile(tmp_path / "weights.bin")
    elif case == "gqa":
        shape = [4, 8, 2, 3, 4, 12]
    (tmp_path / "weights.json").write_text(manifest_text(shape, name, **kw))
    with pytest.raises(qd.QdError) as e:
        qd.bundle_read_layer(str(tmp_path / "weights.json"))
    assert needle in str(e.value)


def test_tail_round_trip_known_answer(tmp_path):
    # tests/qwen_weight_bundle.cpp:186-211.
    emb = np.array([1, 2, 3, 4, 0.5, 0.6, 0.7, 0.8], np.float32)
    norm = np.array([5, 6, 7, 8], np.float32)
    head = np.array([0, .1, .2, .3, 1, 1.1, 1.2, 1.3, 2, 2.1, 2.2, 2.3], np.float32)
    m = str(tmp_path / "tail.json")
    qd.bundle_write_tail(m, "tail.bin", 4, 3, [2, 1], emb, norm, head)
    h, v, ids, t = qd.bundle_read_tail(m)
    assert (h, v, list(ids)) == (4, 3, [2, 1])
    assert np.array_equal(t, np.concatenate([emb, norm, head]))


def test_layer_bytes_identical_to_reference_writer(tmp_path):
    lib = ref_lib()
    shape = np.array([16, 64, 4, 2, 16, 96], np.uint32)
    data = np.random.default_rng(0).standard_normal(sum(counts(shape))).astype(np.float32)
    (tmp_path / "a").mkdir()
    (tmp_path / "b").mkdir()
    ma, mb = str(tmp_path / "a" / "weights.json"), str(tmp_path / "b" / "weights.json")
    qd.bundle_write_layer(ma, "weights.bin", shape, 1e6, data)
    assert lib.ref_write_layer(mb.encode(), b"weights.bin", up(shape), 1e6, fp(data)) == 0
    assert open(ma, "rb").read() == open(mb, "rb").read()
    assert (tmp_path / "a" / "weights.bin").read_bytes() == (tmp_path / "b" / "weights.bin").read_bytes()


def test_cross_read_layer_both_directions(tmp_path):
    lib = ref_lib()
    shape = np.array([8, 32, 2, 1, 16, 48], np.uint32)
    data = np.random.default_rng(1).standard_normal(sum(counts(shape))).astype(np.float32)
    m = str(tmp_path / "mine.json")
    qd.bundle_write_layer(m, "mine.bin", shape, 10000.0, data)
    s6 = np.zeros(6, np.uint32)
    theta = C.c_float()
    out = np.empty(data.size, np.float32)
    assert lib.ref_load_layer(m.encode(), up(s6), C.byref(theta), fp(out), out.size) == data.size
    assert np.array_equal(out, data) and list(s6) == list(shape) and theta.value == 10000.0
    r = str(tmp_path / "ref.json")
    assert lib.ref_write_layer(r.encode(), b"ref.bin", up(shape), 2.5e5, fp(data)) == 0
    shape2, theta2, t2 = qd.bundle_read_layer(r)
    assert np.array_equal(t2, data) and list(shape2) == list(shape) and theta2 == 2.5e5


def test_cross_read_tail_both_directions(tmp_path):
    lib = ref_lib()
    hidden, vocab = 16, 10
    ids = np.array([3, 1, 4, 1, 5], np.uint32)
    rng = np.random.default_rng(2)
    emb = rng.standard_normal(ids.size * hidden).astype(np.float32)
    norm = rng.standard_normal(hidden).astype(np.float32)
    head = rng.standard_normal(vocab * hidden).astype(np.float32)
    m = str(tmp_path / "mine.json")
    qd.bundle_write_tail(m, "mine.bin", hidden, vocab, ids, emb, norm, head)
    h, v, n = C.c_uint32(), C.c_uint32(), C.c_size_t()
    rid = np.empty(16, np.uint32)
    out = np.empty(emb.size + norm.size + head.size, np.float32)
    assert lib.ref_load_tail(m.encode(), C.byref(h), C.byref(v), up(rid), 16, C.byref(n), fp(out),
                             out.size) == out.size
    assert (h.value, v.value, list(rid[:n.value])) == (hidden, vocab, list(ids))
    assert np.array_equal(out, np.concatenate([emb, norm, head]))
    r = str(tmp_path / "ref.json")
    assert lib.ref_write_tail(r.encode(), b"ref.bin", hidden, vocab, up(ids), ids.size, fp(emb), fp(norm),
                              fp(head)) == 0
    assert open(r, "rb").read() == open(m.replace("mine.json", "mine.json"), "rb").read().replace(
        b"mine.bin", b"ref.bin")
    h2, v2, ids2, t2 = qd.bundle_read_tail(r)
    assert (h2, v2, list(ids2)) == (hidden, vocab, list(ids))
    assert np.array_equal(t2, np.concatenate([emb, norm, head]))


def test_reference_rejects_what_we_reject(tmp_path):
    """Same inputs, same verdicts: each malformed manifest fails in both readers."""
    lib = ref_lib()
    data = known_answer_data(SHAPE)
    data.tofile(tmp_path / "weights.bin")
    for kw, name in [({"skip": "q_bias"}, "weights.bin"), ({}, "../x.bin"), ({"dtype": "f16"}, "weights.bin")]:
        (tmp_path / "m.json").write_text(manifest_text(SHAPE, name, **kw))
        with pytest.raises(qd.QdError):
            qd.bundle_read_layer(str(tmp_path / "m.json"))
        s6 = np.zeros(6, np.uint32)
        theta = C.c_float()
        out = np.empty(data.size, np.float32)
        assert lib.ref_load_layer(str(tmp_path / "m.json").encode(), up(s6), C.byref(theta), fp(out),
                                  out.size) == -1
