"""ctypes binding of the CPU oracle (oracle/libqwen_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
CPU-baseline leg of bench.py, as the checker. The product path never uses it.
The C sources name the reference file:line each function restates.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libqwen_oracle.so")

ATTN_NORM, MLP_NORM, Q_W, K_W, V_W, Q_B, K_B, V_B, O_W, GATE_W, UP_W, DOWN_W = range(12)
LAYER_TENSORS = 12
EMBED, FINAL_NORM, LM_HEAD = 0x100, 0x101, 0x102


class Shape(C.Structure):
    _fields_ = [
        ("hidden", C.c_uint32),
        ("heads", C.c_uint32),
        ("kv_heads", C.c_uint32),
        ("head_dim", C.c_uint32),
        ("intermediate", C.c_uint32),
        ("vocab", C.c_uint32),
        ("layers", C.c_uint32),
        ("eps", C.c_float),
        ("rope_theta", C.c_float),
    ]


@dataclass(frozen=True)
class ModelShape:
    hidden: int = 896
    heads: int = 14
    kv_heads: int = 2
    head_dim: int = 64
    intermediate: int = 4864
    vocab: int = 151936
    layers: int = 24
    eps: float = 1e-6
    rope_theta: float = 1e6

    def c(self) -> Shape:
        return Shape(self.hidden, self.heads, self.kv_heads, self.head_dim,
                     self.intermediate, self.vocab, self.layers, self.eps,
                     self.rope_theta)


QWEN25_05B = ModelShape()

_F = C.POINTER(C.c_float)
_U = C.POINTER(C.c_uint32)


def _load():
    if not os.path.exists(_LIB_PATH):
        raise RuntimeError(f"oracle library missing: {_LIB_PATH} (run make -C oracle)")
    lib = C.CDLL(_LIB_PATH)
    sig = {
        "qo_rng_u64": (C.c_uint64, [C.c_uint64, C.c_uint64, C.c_uint64]),
        "qo_rng_normal": (C.c_double, [C.c_uint64, C.c_uint64, C.c_uint64]),
        "qo_fill_normal": (None, [_F, C.c_size_t, C.c_uint64, C.c_uint64, C.c_float, C.c_float]),
        "qo_fill_tokens": (None, [_U, C.c_size_t, C.c_uint64, C.c_uint64, C.c_uint32]),
        "qo_layer_stream": (C.c_uint64, [C.c_uint32, C.c_uint32]),
        "qo_tail_stream": (C.c_uint64, [C.c_uint32]),
        "qo_model_create": (C.c_void_p, [C.POINTER(Shape), C.c_int]),
        "qo_model_destroy": (None, [C.c_void_p]),
        "qo_model_tensor": (_F, [C.c_void_p, C.c_uint32, C.c_uint32, C.POINTER(C.c_size_t)]),
        "qo_model_fill_synthetic": (None, [C.c_void_p, C.c_uint64, C.c_float, C.c_float, C.c_float]),
        "qo_cache_create": (C.c_void_p, [C.c_void_p, C.c_uint32]),
        "qo_cache_destroy": (None, [C.c_void_p]),
        "qo_cache_layer": (_F, [C.c_void_p, C.c_uint32, C.c_int]),
        "qo_rmsnorm": (None, [_F, _F, C.c_uint32, C.c_float, _F]),
        "qo_gemv": (None, [_F, _F, _F, C.c_uint32, C.c_uint32, _F]),
        "qo_rope_tables": (None, [C.c_float, C.c_uint32, C.c_uint32, _F, _F]),
        "qo_rope_apply": (None, [_F, C.c_uint32, C.c_uint32, _F, _F]),
        "qo_attention": (None, [_F, _F, _F, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, _F]),
        "qo_silu_mul": (C.c_float, [C.c_float, C.c_float]),
        "qo_argmax": (C.c_uint32, [_F, C.c_uint32, _F]),
        "qo_layer_step": (None, [C.c_void_p, C.c_uint32, _F, _F, _F, C.c_uint32, _F, _F]),
        "qo_decode_step": (C.c_uint32, [C.c_void_p, C.c_void_p, C.c_uint32, C.c_uint32, _F, _F]),
        "qo_last_final_normed": (_F, [C.c_void_p]),
        "qo_prefill": (C.c_uint32, [C.c_void_p, C.c_void_p, _U, C.c_uint32, C.c_uint32, _F, _F]),
        "qo_threads": (C.c_int, []),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


def fptr(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_F)


def uptr(a: np.ndarray):
    assert a.dtype == np.uint32 and a.flags.c_contiguous
    return a.ctypes.data_as(_U)


def rng_u64(seed: int, stream: int, counter: int) -> int:
    return lib.qo_rng_u64(seed, stream, counter)


def rng_normal(seed: int, stream: int, index: int) -> float:
    return lib.qo_rng_normal(seed, stream, index)


def fill_normal(count: int, seed: int, stream: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(count, np.float32)
    lib.qo_fill_normal(fptr(out), count, seed, stream, mean, std)
    return out


def fill_tokens(count: int, seed: int, stream: int, vocab: int) -> np.ndarray:
    out = np.empty(count, np.uint32)
    lib.qo_fill_tokens(uptr(out), count, seed, stream, vocab)
    return out


def layer_stream(layer: int, kind: int) -> int:
    return lib.qo_layer_stream(layer, kind)


def tail_stream(kind: int) -> int:
    return lib.qo_tail_stream(kind)


def rmsnorm(x: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    out = np.empty_like(x)
    lib.qo_rmsnorm(fptr(x), fptr(w), x.size, eps, fptr(out))
    return out


def gemv(w: np.ndarray, x: np.ndarray, bias: np.ndarray | None = None) -> np.ndarray:
    w = np.ascontiguousarray(w, np.float32)
    x = np.ascontiguousarray(x, np.float32)
    rows, cols = w.shape
    y = np.empty(rows, np.float32)
    b = None if bias is None else np.ascontiguousarray(bias, np.float32)
    lib.qo_gemv(fptr(w), fptr(x), None if b is None else fptr(b), rows, cols, fptr(y))
    return y


def rope_tables(theta: float, head_dim: int, positions: int):
    half = head_dim // 2
    cos = np.empty((positions, half), np.float32)
    sin = np.empty((positions, half), np.float32)
    lib.qo_rope_tables(theta, head_dim, positions, fptr(cos), fptr(sin))
    return cos, sin


def rope_apply(vec: np.ndarray, head_dim: int, cos_row: np.ndarray, sin_row: np.ndarray) -> np.ndarray:
    v = np.array(vec, np.float32, copy=True)
    c = np.ascontiguousarray(cos_row, np.float32)
    s = np.ascontiguousarray(sin_row, np.float32)
    lib.qo_rope_apply(fptr(v), v.size // head_dim, head_dim, fptr(c), fptr(s))
    return v


def attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, heads: int, kv_heads: int, head_dim: int) -> np.ndarray:
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    length = k.size // (kv_heads * head_dim)
    out = np.empty(heads * head_dim, np.float32)
    lib.qo_attention(fptr(q), fptr(k), fptr(v), heads, kv_heads, head_dim, length, fptr(out))
    return out


def silu_mul(g: float, u: float) -> float:
    return lib.qo_silu_mul(g, u)


def argmax(values: np.ndarray) -> tuple[int, float]:
    v = np.ascontiguousarray(values, np.float32)
    best = C.c_float()
    idx = lib.qo_argmax(fptr(v), v.size, C.byref(best))
    return int(idx), float(best.value)


class Model:
    """Host FP32 model; synthetic fill follows the shared generator spec."""

    def __init__(self, shape: ModelShape = QWEN25_05B, tied: bool = True):
        self.shape = shape
        self._c_shape = shape.c()
        self.tied = tied
        self.handle = lib.qo_model_create(C.byref(self._c_shape), 1 if tied else 0)
        if not self.handle:
            raise MemoryError("qo_model_create failed")

    def close(self):
        if self.handle:
            lib.qo_model_destroy(self.handle)
            self.handle = None

    def __del__(self):
        self.close()

    def tensor(self, layer: int, kind: int) -> np.ndarray:
        n = C.c_size_t()
        p = lib.qo_model_tensor(self.handle, layer, kind, C.byref(n))
        if not p:
            raise KeyError((layer, kind))
        return np.ctypeslib.as_array(p, shape=(n.value,))

    def fill_synthetic(self, seed: int, weight_std: float = 0.02, bias_std: float = 0.01, norm_gain: float = 1.0):
        lib.qo_model_fill_synthetic(self.handle, seed, weight_std, bias_std, norm_gain)


class Cache:
    def __init__(self, model: Model, capacity: int):
        self.model = model
        self.capacity = capacity
        self.handle = lib.qo_cache_create(model.handle, capacity)
        if not self.handle:
            raise MemoryError("qo_cache_create failed")
        s = model.shape
        self.kv_dim = s.kv_heads * s.head_dim
        self.cos, self.sin = rope_tables(s.rope_theta, s.head_dim, capacity)

    def close(self):
        if self.handle:
            lib.qo_cache_destroy(self.handle)
            self.handle = None

    def __del__(self):
        self.close()

    def layer(self, layer: int, value: bool) -> np.ndarray:
        p = lib.qo_cache_layer(self.handle, layer, 1 if value else 0)
        return np.ctypeslib.as_array(p, shape=(self.capacity, self.kv_dim))

    def final_normed(self) -> np.ndarray:
        p = lib.qo_last_final_normed(self.handle)
        return np.ctypeslib.as_array(p, shape=(self.model.shape.hidden,)).copy()

    def decode_step(self, token: int, position: int, want_logits: bool = True):
        logits = np.empty(self.model.shape.vocab, np.float32) if want_logits else None
        top = C.c_float()
        tok = lib.qo_decode_step(self.model.handle, self.handle, token, position,
                                 None if logits is None else fptr(logits), C.byref(top))
        return int(tok), float(top.value), logits

    def prefill(self, tokens, start: int = 0, want_logits: bool = True):
        t = np.ascontiguousarray(tokens, np.uint32)
        logits = np.empty(self.model.shape.vocab, np.float32) if want_logits else None
        top = C.c_float()
        tok = lib.qo_prefill(self.model.handle, self.handle, uptr(t), t.size, start,
                             None if logits is None else fptr(logits), C.byref(top))
        return int(tok), float(top.value), logits

    def layer_step(self, layer: int, hidden: np.ndarray, position: int) -> np.ndarray:
        h = np.array(hidden, np.float32, copy=True)
        k = self.layer(layer, False)
        v = self.layer(layer, True)
        lib.qo_layer_step(self.model.handle, layer, fptr(h), k.ctypes.data_as(_F),
                          v.ctypes.data_as(_F), position, fptr(self.cos), fptr(self.sin))
        return h


def threads() -> int:
    return int(lib.qo_threads())
