"""Python binding of the MI355X Qwen2 decode engine (libqwen_decode.so).

A thin ctypes mirror of include/qd/qwen_decode.h for tests, the benchmark and
scripting. The engine itself is C++ and HIP; nothing here computes. Every
call raises QdError on a non-success status, so a missing library or GPU
fails loudly instead of falling back to anything.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libqwen_decode.so")
HEADER = os.path.join(_HERE, "..", "include", "qd", "qwen_decode.h")

SUCCESS, INVALID_ARGUMENT, NOT_INITIALIZED, ALREADY_INITIALIZED, NOT_SUPPORTED, RUNTIME, DEVICE_FAULT = range(7)
STOP_NONE, STOP_MAXIMUM_TOKENS, STOP_EOS_TOKEN = range(3)
NO_EOS = 0xFFFFFFFF
EMBED, FINAL_NORM, LM_HEAD = 0x100, 0x101, 0x102
DTYPE_F32, DTYPE_BF16, DTYPE_F16 = 0, 1, 2


class QdError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"qd status {status}: {message}")
        self.status = status


class Config(C.Structure):
    _fields_ = [
        ("hidden", C.c_uint32), ("heads", C.c_uint32), ("kv_heads", C.c_uint32),
        ("head_dim", C.c_uint32), ("intermediate", C.c_uint32), ("vocab", C.c_uint32),
        ("layers", C.c_uint32), ("capacity", C.c_uint32), ("max_batch", C.c_uint32),
        ("tied_lm_head", C.c_uint32), ("rms_eps", C.c_float), ("rope_theta", C.c_float),
        ("device", C.c_int32), ("decoder_dtype", C.c_uint32),
    ]


class SyntheticInit(C.Structure):
    _fields_ = [("weight_std", C.c_float), ("bias_std", C.c_float),
                ("norm_gain", C.c_float), ("reserved", C.c_float)]


class DecodeState(C.Structure):
    _fields_ = [("token_position", C.c_uint32), ("kv_length", C.c_uint32),
                ("sampled_token", C.c_uint32), ("eos_token", C.c_uint32),
                ("generated_tokens", C.c_uint32), ("maximum_tokens", C.c_uint32),
                ("stop_reason", C.c_uint32), ("sampled_logit", C.c_float)]


class Timing(C.Structure):
    _fields_ = [("total_us", C.c_double), ("per_token_us", C.c_double),
                ("tokens", C.c_uint32), ("reserved", C.c_uint32)]


class KernelStat(C.Structure):
    _fields_ = [("name", C.c_char * 48), ("launches", C.c_uint32), ("reserved", C.c_uint32),
                ("total_us", C.c_double), ("bytes", C.c_double), ("flops", C.c_double)]


_F = C.POINTER(C.c_float)
_U = C.POINTER(C.c_uint32)
_E = C.c_void_p

_SIGNATURES = {
    "qd_status_string": (C.c_char_p, [C.c_int]),
    "qd_last_error": (C.c_char_p, []),
    "qd_abi_version": (C.c_uint32, []),
    "qd_device_count": (C.c_int, [_U]),
    "qd_engine_create": (C.c_int, [C.POINTER(Config), C.POINTER(_E)]),
    "qd_engine_destroy": (C.c_int, [_E]),
    "qd_engine_config": (C.c_int, [_E, C.POINTER(Config)]),
    "qd_engine_device_bytes": (C.c_int, [_E, C.POINTER(C.c_uint64)]),
    "qd_engine_resident_grid": (C.c_int, [_E, _U]),
    "qd_load_bundle": (C.c_int, [_E, C.c_char_p]),
    "qd_load_synthetic": (C.c_int, [_E, C.c_uint64, C.POINTER(SyntheticInit)]),
    "qd_read_weight": (C.c_int, [_E, C.c_uint32, C.c_uint32, _F, C.c_size_t]),
    "qd_kv_reset": (C.c_int, [_E, C.c_uint32, C.c_uint32]),
    "qd_write_kv": (C.c_int, [_E, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, _F, _F]),
    "qd_read_kv": (C.c_int, [_E, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32, _F, _F]),
    "qd_read_decode_state": (C.c_int, [_E, C.c_uint32, C.POINTER(DecodeState)]),
    "qd_read_activation": (C.c_int, [_E, C.c_uint32, C.c_uint32, _F, C.c_size_t]),
    "qd_layer_step": (C.c_int, [_E, C.c_uint32, C.c_uint32, _F]),
    "qd_load_hidden": (C.c_int, [_E, C.c_uint32, _F]),
    "qd_embed_hidden": (C.c_int, [_E, C.c_uint32, C.c_uint32]),
    "qd_layer_decode": (C.c_int, [_E, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32]),
    "qd_tail": (C.c_int, [_E, C.c_uint32, _F, _U, _F]),
    "qd_read_logits": (C.c_int, [_E, C.c_uint32, _F, C.c_size_t]),
    "qd_step": (C.c_int, [_E, C.c_uint32, C.c_uint32, _F, _U, _F]),
    "qd_step_graph": (C.c_int, [_E, C.c_uint32, C.c_uint32, _F, _U, _F]),
    "qd_prefill": (C.c_int, [_E, C.c_uint32, _U, C.c_uint32, _F, _U, _F]),
    "qd_step_batch": (C.c_int, [_E, C.c_uint32, _U, _U, _F, _U]),
    "qd_step_batch_noalloc": (C.c_int, [_E, C.c_uint32, _U, _U, _F, _U]),
    "qd_generate_resident": (C.c_int, [_E, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32,
                                       _U, _U, _U, _F]),
    "qd_last_timing": (C.c_int, [_E, C.POINTER(Timing)]),
    "qd_profile_kernels": (C.c_int, [_E, C.c_uint32, C.c_uint32, C.c_uint32, C.POINTER(KernelStat),
                                     C.c_uint32, _U]),
    "qd_profile_batch": (C.c_int, [_E, C.c_uint32, _U, _U, C.c_uint32, C.POINTER(KernelStat),
                                   C.c_uint32, _U]),
    "qd_profile_prefill": (C.c_int, [_E, C.c_uint32, _U, C.c_uint32, C.POINTER(KernelStat),
                                     C.c_uint32, _U]),
    "qd_profile_resident": (C.c_int, [_E, C.c_uint32, C.c_uint32, C.c_uint32, C.POINTER(C.c_double),
                                      C.c_uint32, _U]),
    "qd_trace_resident": (C.c_int, [_E, C.c_uint32, C.c_uint32, C.c_uint32, C.c_uint32,
                                    C.POINTER(C.c_uint64), C.c_size_t, _U, _U, _U]),
    "qd_sync": (C.c_int, [_E]),
    "qd_probe_hbm": (C.c_int, [C.c_int32, C.c_uint64, C.c_uint32, C.POINTER(C.c_double),
                               C.POINTER(C.c_double)]),
    "qd_bundle_write_layer": (C.c_int, [C.c_char_p, C.c_char_p, _U, C.c_float, _F]),
    "qd_bundle_read_layer": (C.c_int, [C.c_char_p, _U, _F, _F, C.c_size_t, C.POINTER(C.c_size_t)]),
    "qd_bundle_write_tail": (C.c_int, [C.c_char_p, C.c_char_p, C.c_uint32, C.c_uint32, _U,
                                       C.c_size_t, _F, _F, _F]),
    "qd_bundle_read_tail": (C.c_int, [C.c_char_p, _U, _U, _U, C.c_size_t, C.POINTER(C.c_size_t),
                                      _F, C.c_size_t, C.POINTER(C.c_size_t)]),
}

_lib = None


def lib():
    """Loads the engine library (raises if it is not built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise QdError(NOT_INITIALIZED, f"engine library missing: {LIB_PATH} (run make -C light-rocm-runtime_amd)")
        handle = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def _check(status: int):
    if status != SUCCESS:
        raise QdError(status, lib().qd_last_error().decode(errors="replace"))


def _f(a: np.ndarray | None):
    if a is None:
        return None
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_F)


def _u(a: np.ndarray | None):
    if a is None:
        return None
    assert a.dtype == np.uint32 and a.flags.c_contiguous
    return a.ctypes.data_as(_U)


def device_count() -> int:
    n = C.c_uint32()
    _check(lib().qd_device_count(C.byref(n)))
    return int(n.value)


def probe_hbm(device: int = 0, nbytes: int = 1 << 31, iters: int = 5):
    """(read GB/s, copy GB/s): best-of-iters streaming read / copy bandwidth."""
    r, c = C.c_double(), C.c_double()
    _check(lib().qd_probe_hbm(device, nbytes, iters, C.byref(r), C.byref(c)))
    return float(r.value), float(c.value)


def status_string(status: int) -> str:
    return lib().qd_status_string(status).decode()


@dataclass
class EngineConfig:
    hidden: int = 896
    heads: int = 14
    kv_heads: int = 2
    head_dim: int = 64
    intermediate: int = 4864
    vocab: int = 151936
    layers: int = 24
    capacity: int = 1024
    max_batch: int = 1
    tied_lm_head: bool = True
    rms_eps: float = 1e-6
    rope_theta: float = 1e6
    device: int = 0
    decoder_dtype: str = "f32"  # "f32", "bf16" or "f16": storage of the decoder layers' matrices

    def c(self) -> Config:
        dtypes = {"f32": DTYPE_F32, "bf16": DTYPE_BF16, "f16": DTYPE_F16}
        if self.decoder_dtype not in dtypes:
            raise ValueError(f"decoder_dtype must be one of {sorted(dtypes)}")
        return Config(self.hidden, self.heads, self.kv_heads, self.head_dim, self.intermediate,
                      self.vocab, self.layers, self.capacity, self.max_batch,
                      1 if self.tied_lm_head else 0, self.rms_eps, self.rope_theta, self.device,
                      dtypes[self.decoder_dtype])


class Engine:
    """Owns one qd_engine. Methods mirror the C entry points one to one."""

    def __init__(self, config: EngineConfig | None = None, **overrides):
        self.config = config or EngineConfig(**overrides)
        self.handle = _E()
        cfg = self.config.c()
        _check(lib().qd_engine_create(C.byref(cfg), C.byref(self.handle)))
        self.kv_dim = self.config.kv_heads * self.config.head_dim

    def close(self):
        if self.handle:
            _check(lib().qd_engine_destroy(self.handle))
            self.handle = _E()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def device_bytes(self) -> int:
        n = C.c_uint64()
        _check(lib().qd_engine_device_bytes(self.handle, C.byref(n)))
        return int(n.value)

    def resident_grid(self) -> int:
        g = C.c_uint32()
        _check(lib().qd_engine_resident_grid(self.handle, C.byref(g)))
        return int(g.value)

    def load_synthetic(self, seed: int, weight_std: float = 0.02, bias_std: float = 0.01,
                       norm_gain: float = 1.0):
        init = SyntheticInit(weight_std, bias_std, norm_gain, 0.0)
        _check(lib().qd_load_synthetic(self.handle, seed, C.byref(init)))

    def load_bundle(self, directory: str):
        _check(lib().qd_load_bundle(self.handle, directory.encode()))

    def read_weight(self, layer: int, kind: int, count: int) -> np.ndarray:
        out = np.empty(count, np.float32)
        _check(lib().qd_read_weight(self.handle, layer, kind, _f(out), count))
        return out

    def kv_reset(self, seq: int, position: int):
        _check(lib().qd_kv_reset(self.handle, seq, position))

    def write_kv(self, seq: int, layer: int, start: int, k: np.ndarray, v: np.ndarray):
        k = np.ascontiguousarray(k, np.float32)
        v = np.ascontiguousarray(v, np.float32)
        count = k.size // self.kv_dim
        _check(lib().qd_write_kv(self.handle, seq, layer, start, count, _f(k), _f(v)))

    def read_kv(self, seq: int, layer: int, start: int, count: int):
        k = np.empty((count, self.kv_dim), np.float32)
        v = np.empty((count, self.kv_dim), np.float32)
        _check(lib().qd_read_kv(self.handle, seq, layer, start, count, _f(k), _f(v)))
        return k, v

    def read_activation(self, seq: int, which: int) -> np.ndarray:
        c = self.config
        n = [c.hidden, c.heads * c.head_dim, c.heads * c.head_dim, c.intermediate][which]
        out = np.empty(n, np.float32)
        _check(lib().qd_read_activation(self.handle, seq, which, _f(out), n))
        return out

    def decode_state(self, seq: int) -> DecodeState:
        s = DecodeState()
        _check(lib().qd_read_decode_state(self.handle, seq, C.byref(s)))
        return s

    def layer_step(self, seq: int, layer: int, hidden: np.ndarray) -> np.ndarray:
        h = np.array(hidden, np.float32, copy=True)
        _check(lib().qd_layer_step(self.handle, seq, layer, _f(h)))
        return h

    def load_hidden(self, seq: int, hidden: np.ndarray):
        h = np.ascontiguousarray(hidden, np.float32)
        assert h.size == self.config.hidden
        _check(lib().qd_load_hidden(self.handle, seq, _f(h)))

    def embed_hidden(self, seq: int, token: int):
        _check(lib().qd_embed_hidden(self.handle, seq, token))

    def layer_decode(self, seq: int, first_layer: int, layer_count: int, valid_keys: int):
        _check(lib().qd_layer_decode(self.handle, seq, first_layer, layer_count, valid_keys))

    def tail(self, seq: int, want_logits: bool = True):
        logits = np.empty(self.config.vocab, np.float32) if want_logits else None
        tok = C.c_uint32()
        top = C.c_float()
        _check(lib().qd_tail(self.handle, seq, _f(logits), C.byref(tok), C.byref(top)))
        return int(tok.value), float(top.value), logits

    def read_logits(self, seq: int) -> np.ndarray:
        out = np.empty(self.config.vocab, np.float32)
        _check(lib().qd_read_logits(self.handle, seq, _f(out), out.size))
        return out

    def step(self, seq: int, token: int, want_logits: bool = True):
        logits = np.empty(self.config.vocab, np.float32) if want_logits else None
        tok = C.c_uint32()
        top = C.c_float()
        _check(lib().qd_step(self.handle, seq, token, _f(logits), C.byref(tok), C.byref(top)))
        return int(tok.value), float(top.value), logits

    def step_graph(self, seq: int, token: int, want_logits: bool = True):
        """qd_step replayed from the slot's captured HIP graph."""
        logits = np.empty(self.config.vocab, np.float32) if want_logits else None
        tok = C.c_uint32()
        top = C.c_float()
        _check(lib().qd_step_graph(self.handle, seq, token, _f(logits), C.byref(tok), C.byref(top)))
        return int(tok.value), float(top.value), logits

    def prefill(self, seq: int, tokens, want_logits: bool = True):
        t = np.ascontiguousarray(tokens, np.uint32)
        logits = np.empty(self.config.vocab, np.float32) if want_logits else None
        tok = C.c_uint32()
        top = C.c_float()
        _check(lib().qd_prefill(self.handle, seq, _u(t), t.size, _f(logits), C.byref(tok), C.byref(top)))
        return int(tok.value), float(top.value), logits

    def step_batch(self, seq_ids, tokens, want_logits: bool = True):
        s = np.ascontiguousarray(seq_ids, np.uint32)
        t = np.ascontiguousarray(tokens, np.uint32)
        logits = np.empty((s.size, self.config.vocab), np.float32) if want_logits else None
        greedy = np.empty(s.size, np.uint32)
        _check(lib().qd_step_batch(self.handle, s.size, _u(s), _u(t), _f(logits), _u(greedy)))
        return greedy, logits

    def step_batch_noalloc(self, seq_ids, tokens, want_logits: bool = True):
        """qd_step_batch_noalloc: one group of up to 16 sequences, scratch in
        the library's static device workspace."""
        s = np.ascontiguousarray(seq_ids, np.uint32)
        t = np.ascontiguousarray(tokens, np.uint32)
        logits = np.empty((s.size, self.config.vocab), np.float32) if want_logits else None
        greedy = np.empty(s.size, np.uint32)
        _check(lib().qd_step_batch_noalloc(self.handle, s.size, _u(s), _u(t), _f(logits), _u(greedy)))
        return greedy, logits

    def generate(self, seq: int, first_token: int, max_tokens: int, eos: int = NO_EOS,
                 want_logits: bool = False):
        out = np.zeros(max_tokens, np.uint32)
        n = C.c_uint32()
        reason = C.c_uint32()
        logits = np.empty((max_tokens, self.config.vocab), np.float32) if want_logits else None
        _check(lib().qd_generate_resident(self.handle, seq, first_token, max_tokens, eos, _u(out),
                                          C.byref(n), C.byref(reason), _f(logits)))
        k = int(n.value)
        return out[:k], int(reason.value), (None if logits is None else logits[:k])

    @staticmethod
    def _stats(call) -> dict:
        cap = 64
        stats = (KernelStat * cap)()
        n = C.c_uint32()
        _check(call(stats, cap, C.byref(n)))
        return {s.name.decode(): (int(s.launches), s.total_us / s.launches, s.bytes / s.launches,
                                  s.flops / s.launches) for s in stats[:n.value]}

    def profile_kernels(self, seq: int, first_token: int, tokens: int) -> dict:
        """Per-kernel {name: (launches, avg_us, avg_bytes, avg_flops)} over
        `tokens` stream-ordered steps."""
        return self._stats(lambda st, cap, n: lib().qd_profile_kernels(
            self.handle, seq, first_token, tokens, st, cap, n))

    def profile_batch(self, seq_ids, tokens, steps: int) -> dict:
        """Per-kernel {name: (launches, avg_us, avg_bytes, avg_flops)} over
        `steps` batched steps of the listed slots."""
        s = np.ascontiguousarray(seq_ids, np.uint32)
        t = np.ascontiguousarray(tokens, np.uint32)
        return self._stats(lambda st, cap, n: lib().qd_profile_batch(
            self.handle, s.size, _u(s), _u(t), steps, st, cap, n))

    def profile_prefill(self, seq: int, tokens) -> dict:
        """Per-kernel {name: (launches, avg_us, avg_bytes, avg_flops)} of one
        prefill of `tokens` into the slot (which advances as qd_prefill)."""
        t = np.ascontiguousarray(tokens, np.uint32)
        return self._stats(lambda st, cap, n: lib().qd_profile_prefill(
            self.handle, seq, _u(t), t.size, st, cap, n))

    RESIDENT_STAGES = tuple(f"{s}.{k}" for s in ("qkv", "attention", "oproj", "gateup", "down",
                                                  "lmhead", "argmax") for k in ("wait", "work")) + \
        ("attention.stage", "attention.math", "attention.emit")

    def profile_resident(self, seq: int, first_token: int, tokens: int) -> dict:
        """Per-stage microseconds (summed over `tokens`) of the resident kernel."""
        out = (C.c_double * 32)()
        n = C.c_uint32()
        _check(lib().qd_profile_resident(self.handle, seq, first_token, tokens, out, 32, C.byref(n)))
        return {name: out[i] for i, name in enumerate(self.RESIDENT_STAGES[:n.value])}

    def trace_resident(self, seq: int, first_token: int, tokens: int, trace_token: int) -> np.ndarray:
        """Timeline [workgroup, layer row, stage] (microseconds from the earliest
        stamp) of token `trace_token` in a profiled resident launch; 0 = no stamp."""
        g, r, st = C.c_uint32(), C.c_uint32(), C.c_uint32()
        cap = max(self.resident_grid(), 1) * (self.config.layers + 1) * len(self.RESIDENT_STAGES)
        buf = np.zeros(cap, np.uint64)
        _check(lib().qd_trace_resident(self.handle, seq, first_token, tokens, trace_token,
                                       buf.ctypes.data_as(C.POINTER(C.c_uint64)), cap,
                                       C.byref(g), C.byref(r), C.byref(st)))
        t = buf[: g.value * r.value * st.value].reshape(g.value, r.value, st.value).astype(np.float64)
        stamped = t > 0
        if stamped.any():
            t[stamped] = (t[stamped] - t[stamped].min()) / 100.0
        return t

    def last_timing(self) -> Timing:
        t = Timing()
        _check(lib().qd_last_timing(self.handle, C.byref(t)))
        return t

    def sync(self):
        _check(lib().qd_sync(self.handle))


# ---- bundle I/O (host only) -----------------------------------------------------

def bundle_write_layer(manifest: str, data_name: str, shape6, rope_theta: float, tensors: np.ndarray):
    s = np.ascontiguousarray(shape6, np.uint32)
    t = np.ascontiguousarray(tensors, np.float32)
    _check(lib().qd_bundle_write_layer(manifest.encode(), data_name.encode(), _u(s), rope_theta, _f(t)))


def bundle_read_layer(manifest: str, capacity: int = 1 << 26):
    shape = np.zeros(6, np.uint32)
    theta = C.c_float()
    count = C.c_size_t()
    buf = np.empty(capacity, np.float32)
    _check(lib().qd_bundle_read_layer(manifest.encode(), _u(shape), C.byref(theta), _f(buf), capacity,
                                      C.byref(count)))
    return shape, float(theta.value), buf[:count.value].copy()


def bundle_write_tail(manifest: str, data_name: str, hidden: int, vocab: int, token_ids,
                      embeddings: np.ndarray, final_norm: np.ndarray, lm_head: np.ndarray):
    ids = np.ascontiguousarray(token_ids, np.uint32)
    _check(lib().qd_bundle_write_tail(manifest.encode(), data_name.encode(), hidden, vocab, _u(ids), ids.size,
                                      _f(np.ascontiguousarray(embeddings, np.float32)),
                                      _f(np.ascontiguousarray(final_norm, np.float32)),
                                      _f(np.ascontiguousarray(lm_head, np.float32))))


def bundle_read_tail(manifest: str, ids_capacity: int = 1 << 20, capacity: int = 1 << 28):
    hidden = C.c_uint32()
    vocab = C.c_uint32()
    n_ids = C.c_size_t()
    count = C.c_size_t()
    ids = np.empty(ids_capacity, np.uint32)
    buf = np.empty(capacity, np.float32)
    _check(lib().qd_bundle_read_tail(manifest.encode(), C.byref(hidden), C.byref(vocab), _u(ids), ids_capacity,
                                     C.byref(n_ids), _f(buf), capacity, C.byref(count)))
    return int(hidden.value), int(vocab.value), ids[:n_ids.value].copy(), buf[:count.value].copy()
