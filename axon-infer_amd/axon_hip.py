"""ctypes binding of the hip kernel table's C ABI (include/axon_hip.h) and of the device-resident
forward pass (include/axon_model.h).

This is the Python face of the library for tests, the benchmark and smoke checks. Device memory
is owned by DeviceBuffer; every call raises HipError with the library's message on a non-zero
status. Nothing here computes on the CPU: if libaxon_hip.so is missing or no gfx950 device is
present, the calls fail loudly.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

PKG = Path(__file__).resolve().parent
HIP_SO = PKG / "libaxon_hip.so"
HOST_SO = PKG / "libaxon_host.so"

F32, F16, Q4_0, Q4_1, Q8_0, Q6_K, BF16 = 0, 1, 2, 3, 8, 14, 30


class HipError(RuntimeError):
    pass


_lib = None


def lib() -> C.CDLL:
    """libaxon_hip.so, loaded once. Raises when it has not been built."""
    global _lib
    if _lib is None:
        if not HIP_SO.exists():
            raise HipError(f"{HIP_SO} is missing: build it with __graft_entry__.build()")
        L = C.CDLL(str(HIP_SO))
        L.axon_hip_last_error.restype = C.c_char_p
        L.axon_hip_attention_scratch_floats.restype = C.c_size_t
        _lib = L
    return _lib


def check(rc: int, what: str = "") -> None:
    if rc != 0:
        raise HipError(f"{what}: status {rc}: {lib().axon_hip_last_error().decode()}")


def device_count() -> int:
    n = C.c_int(0)
    lib().axon_hip_device_count(C.byref(n))
    return n.value


def init(device: int = 0) -> None:
    check(lib().axon_hip_init(device), "axon_hip_init")


def synchronize() -> None:
    check(lib().axon_hip_synchronize(), "synchronize")


def _arg(a):
    if isinstance(a, DeviceBuffer):
        return C.c_void_p(a.ptr)
    if a is None:
        return C.c_void_p(0)
    if isinstance(a, float):
        return C.c_float(a)
    if isinstance(a, (C._SimpleCData, C.c_void_p, C.Array)) or hasattr(a, "_fields_"):
        return a
    if isinstance(a, np.ndarray):
        return C.c_void_p(a.ctypes.data)
    return C.c_size_t(a)


def call(name: str, *args) -> None:
    """Calls axon_hip_<name> with DeviceBuffers as device pointers, ints as size_t, floats
    as float, raising on a non-zero status."""
    check(getattr(lib(), "axon_hip_" + name)(*[_arg(a) for a in args]), name)


class DeviceBuffer:
    """An owned device allocation."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = C.c_void_p(0)
        check(lib().axon_hip_malloc(C.byref(p), C.c_size_t(max(self.nbytes, 1))), "malloc")
        self.ptr = p.value or 0

    @classmethod
    def of(cls, a: np.ndarray) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.upload(a)
        return b

    def upload(self, a: np.ndarray, offset: int = 0) -> None:
        a = np.ascontiguousarray(a)
        assert offset + a.nbytes <= self.nbytes
        check(lib().axon_hip_memcpy_h2d(C.c_void_p(self.ptr + offset), C.c_void_p(a.ctypes.data),
                                         C.c_size_t(a.nbytes)), "memcpy_h2d")

    def download(self, dtype, count: int | None = None, offset: int = 0) -> np.ndarray:
        dt = np.dtype(dtype)
        if count is None:
            count = (self.nbytes - offset) // dt.itemsize
        out = np.empty(count, dtype=dt)
        check(lib().axon_hip_memcpy_d2h(C.c_void_p(out.ctypes.data), C.c_void_p(self.ptr + offset),
                                         C.c_size_t(out.nbytes)), "memcpy_d2h")
        return out

    def fill(self, value: int = 0) -> None:
        check(lib().axon_hip_memset(C.c_void_p(self.ptr), C.c_int(value), C.c_size_t(self.nbytes)), "memset")

    def at(self, offset_bytes: int) -> C.c_void_p:
        return C.c_void_p(self.ptr + offset_bytes)

    def free(self) -> None:
        if self.ptr:
            lib().axon_hip_free(C.c_void_p(self.ptr))
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Event:
    def __init__(self):
        p = C.c_void_p(0)
        check(lib().axon_hip_event_create(C.byref(p)), "event_create")
        self.h = p

    def record(self) -> None:
        check(lib().axon_hip_event_record(self.h), "event_record")

    def elapsed_ms(self, later: "Event") -> float:
        ms = C.c_float(0)
        check(lib().axon_hip_event_elapsed_ms(self.h, later.h, C.byref(ms)), "event_elapsed")
        return ms.value

    def __del__(self):
        try:
            lib().axon_hip_event_destroy(self.h)
        except Exception:
            pass


class RopeRowsArgs(C.Structure):
    _fields_ = [("q", C.c_void_p), ("k", C.c_void_p), ("v", C.c_void_p), ("bq", C.c_void_p), ("bk", C.c_void_p),
                ("bv", C.c_void_p), ("pos", C.c_void_p), ("pos0", C.c_int32), ("q_stride", C.c_uint32),
                ("k_stride", C.c_uint32), ("n_head", C.c_uint32), ("n_kv", C.c_uint32), ("head_dim", C.c_uint32),
                ("rotary_dim", C.c_uint32), ("neox", C.c_int), ("theta", C.c_float), ("freq_factors", C.c_void_p),
                ("table", C.c_void_p), ("cache", C.c_void_p), ("cache_off", C.c_void_p),
                ("k_layer_off", C.c_int64), ("v_layer_off", C.c_int64), ("cache_f16", C.c_int)]


class AttentionRowsArgs(C.Structure):
    _fields_ = [("q", C.c_void_p), ("out", C.c_void_p), ("q_stride", C.c_uint32), ("out_stride", C.c_uint32),
                ("kv", C.c_void_p), ("k_off", C.c_void_p), ("v_off", C.c_void_p), ("n_vis", C.c_void_p),
                ("k_layer_off", C.c_int64), ("v_layer_off", C.c_int64), ("n_past", C.c_int32),
                ("n_head", C.c_uint32), ("n_kv", C.c_uint32), ("head_dim", C.c_uint32), ("scale", C.c_float),
                ("f16", C.c_int), ("scratch", C.c_void_p), ("max_vis", C.c_uint32), ("outq", C.c_void_p)]


class DecodeShape(C.Structure):
    """axon_hip_decode_shape (include/axon_hip.h)."""
    _fields_ = [("n_layer", C.c_uint32), ("n_embd", C.c_uint32), ("n_head", C.c_uint32), ("n_head_kv", C.c_uint32),
                ("n_ff", C.c_uint32), ("rotary_dim", C.c_uint32), ("type_qkv", C.c_int), ("type_o", C.c_int),
                ("type_gate_up", C.c_int), ("type_down", C.c_int), ("max_ctx", C.c_uint32), ("cache_f16", C.c_int)]


class MatvecFusedArgs(C.Structure):
    """axon_hip_matvec_fused_args (include/axon_hip.h)."""
    _fields_ = [("type", C.c_int), ("n_seg", C.c_size_t), ("w", C.c_void_p * 3), ("n_out", C.c_size_t * 3),
                ("n_rows", C.c_size_t), ("n_in", C.c_size_t), ("in_mode", C.c_int), ("xq", C.c_void_p),
                ("x", C.c_void_p), ("x_stride", C.c_size_t), ("norm_w", C.c_void_p), ("eps", C.c_float),
                ("out_mode", C.c_int), ("y", C.c_void_p * 3), ("y_stride", C.c_size_t * 3), ("bias", C.c_void_p * 3),
                ("rope_table", C.c_void_p), ("rot_half", C.c_uint32), ("head_dim", C.c_uint32), ("pos", C.c_void_p),
                ("cache_off", C.c_void_p), ("cache", C.c_void_p), ("k_layer_off", C.c_int64),
                ("v_layer_off", C.c_int64), ("outq", C.c_void_p), ("cache_f16", C.c_int)]


def ptr_of(b) -> int:
    return 0 if b is None else (b.ptr if isinstance(b, DeviceBuffer) else int(b))


# ---------------------------------------------------------------------------------------------
# The device-resident forward pass (libaxon_host.so, include/axon_model.h)

# axon_model_probe's type for the attention launches (AXON_MODEL_PROBE_ATTENTION).
PROBE_ATTENTION = -2
# ... and for the persistent decode kernel's launches alone (AXON_MODEL_PROBE_STEP).
PROBE_STEP = -3


class ModelOptions(C.Structure):
    _fields_ = [("max_seq", C.c_size_t), ("max_ctx", C.c_size_t), ("max_batch", C.c_size_t),
                ("max_caches", C.c_size_t), ("exact_activations", C.c_int), ("kernels", C.c_char_p),
                ("cache_type", C.c_int), ("no_repack", C.c_int), ("no_persistent", C.c_int)]


class ModelInfo(C.Structure):
    _fields_ = [("n_layer", C.c_uint32), ("n_embd", C.c_uint32), ("n_head", C.c_uint32), ("n_head_kv", C.c_uint32),
                ("n_ff", C.c_uint32), ("n_vocab", C.c_uint32), ("head_dim", C.c_uint32), ("rotary_dim", C.c_uint32),
                ("max_seq", C.c_size_t), ("max_ctx", C.c_size_t), ("max_batch", C.c_size_t),
                ("weight_bytes_per_token", C.c_size_t), ("device_bytes", C.c_size_t),
                ("kv_bytes_per_position", C.c_size_t), ("cache_type", C.c_int), ("persistent_decode", C.c_int)]


class SamplerConfig(C.Structure):
    """axon_sampler_config: SamplerConfig (include/axon/sampler.h:10-17) without the seed; the
    defaults are the reference's."""
    _fields_ = [("temperature", C.c_float), ("top_k", C.c_int), ("top_p", C.c_float), ("min_p", C.c_float),
                ("repeat_penalty", C.c_float), ("repeat_last_n", C.c_int)]

    def __init__(self, temperature=0.8, top_k=40, top_p=0.95, min_p=0.05, repeat_penalty=1.1, repeat_last_n=64):
        super().__init__(temperature, top_k, top_p, min_p, repeat_penalty, repeat_last_n)


class Rng(C.Structure):
    """axon_rng: the sampler's generator (src/sampling/rng.h), seeded as the reference seeds it."""
    _fields_ = [("s", C.c_uint64 * 4)]

    def __init__(self, seed: int = 0):
        super().__init__()
        host().axon_rng_seed(C.byref(self), C.c_uint64(seed))

    def next(self) -> int:
        return host().axon_rng_next(C.byref(self))

    def uniform(self) -> float:
        return host().axon_rng_uniform(C.byref(self))

    def state(self):
        return tuple(self.s)


def sample_candidates(config: SamplerConfig, rng: Rng, logits, ids) -> int:
    """The host stages of the sampler alone (axon_sample_candidates) over candidates in top-k order."""
    lg = np.ascontiguousarray(logits, np.float32)
    ix = np.ascontiguousarray(ids, np.int32)
    out = C.c_int32(0)
    _mcheck(host().axon_sample_candidates(C.byref(config), C.byref(rng), lg.ctypes.data, ix.ctypes.data, len(lg),
                                          C.byref(out)), "sample_candidates")
    return out.value


_host = None


def host() -> C.CDLL:
    """libaxon_host.so, loaded once (it links libaxon_hip.so)."""
    global _host
    if _host is None:
        if not HOST_SO.exists():
            raise HipError(f"{HOST_SO} is missing: build it with __graft_entry__.build()")
        lib()
        L = C.CDLL(str(HOST_SO))
        L.axon_model_last_error.restype = C.c_char_p
        L.axon_model_table_name.restype = C.c_char_p
        L.axon_model_table_name.argtypes = [C.c_void_p]
        L.axon_model_load.argtypes = [C.c_char_p, C.POINTER(ModelOptions), C.POINTER(C.c_void_p)]
        L.axon_model_free.argtypes = [C.c_void_p]
        L.axon_model_get_info.argtypes = [C.c_void_p, C.POINTER(ModelInfo)]
        L.axon_model_set_persistent_decode.argtypes = [C.c_void_p, C.c_int]
        L.axon_model_cache_new.argtypes = [C.c_void_p, C.POINTER(C.c_int)]
        L.axon_model_cache_free.argtypes = [C.c_void_p, C.c_int]
        L.axon_model_cache_pos.argtypes = [C.c_void_p, C.c_int, C.POINTER(C.c_size_t)]
        L.axon_model_cache_truncate.argtypes = [C.c_void_p, C.c_int, C.c_size_t]
        L.axon_model_cache_read.argtypes = [C.c_void_p, C.c_int, C.c_size_t, C.c_int, C.c_size_t, C.c_void_p]
        L.axon_model_cache_fill.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_size_t]
        L.axon_model_forward.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p]
        L.axon_model_forward_prefill.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_size_t, C.c_void_p]
        L.axon_model_forward_batch.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p]
        L.axon_model_forward_mixed.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_size_t, C.c_void_p, C.c_void_p,
                                               C.c_size_t, C.c_void_p]
        L.axon_model_generate_greedy.argtypes = [C.c_void_p, C.c_int, C.c_int32, C.c_size_t, C.c_void_p]
        L.axon_model_greedy.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_float, C.c_int, C.c_void_p,
                                        C.c_size_t]
        L.axon_rng_seed.argtypes = [C.c_void_p, C.c_uint64]
        L.axon_rng_seed.restype = None
        L.axon_rng_next.argtypes = [C.c_void_p]
        L.axon_rng_next.restype = C.c_uint64
        L.axon_rng_uniform.argtypes = [C.c_void_p]
        L.axon_rng_uniform.restype = C.c_double
        L.axon_model_sample.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                        C.c_size_t]
        L.axon_sample_candidates.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p]
        L.axon_model_probe.argtypes = [C.c_void_p, C.c_int, C.c_int]
        L.axon_model_probe_read.argtypes = [C.c_void_p, C.POINTER(C.c_double), C.POINTER(C.c_size_t),
                                            C.POINTER(C.c_double)]
        _host = L
    return _host


def _mcheck(rc: int, what: str) -> None:
    if rc != 0:
        raise HipError(f"{what}: status {rc}: {host().axon_model_last_error().decode()}")


class Model:
    """LlamaModel on the hip table (src/model/llama.h:87-110): logits come back as numpy
    arrays [rows, n_vocab]; caches are int slot ids of the device KV pool."""

    CACHE_TYPES = {"f32": 0, "f16": 1}  # CacheType (src/model/config.h:16)

    def __init__(self, path, max_seq=512, max_ctx=4096, max_batch=1, max_caches=0, exact=False, kernels="hip",
                 cache="f32", repack=True, persistent=True):
        if cache not in self.CACHE_TYPES:
            raise ValueError(f"cache type {cache!r}: f32 or f16")
        o = ModelOptions(max_seq, max_ctx, max_batch, max_caches, int(exact), kernels.encode(),
                         self.CACHE_TYPES[cache], int(not repack), int(not persistent))
        h = C.c_void_p(0)
        _mcheck(host().axon_model_load(str(path).encode(), C.byref(o), C.byref(h)), f"load {path}")
        self.h = h
        info = ModelInfo()
        host().axon_model_get_info(self.h, C.byref(info))
        self.info = info
        self.n_vocab = info.n_vocab
        self.table_name = host().axon_model_table_name(self.h).decode()

    def persistent_decode(self) -> bool:
        """Whether one-row cached passes run as the persistent kernel now (a pass whose kernel
        gave up turns it off)."""
        info = ModelInfo()
        host().axon_model_get_info(self.h, C.byref(info))
        return bool(info.persistent_decode)

    def set_persistent_decode(self, on: bool) -> None:
        _mcheck(host().axon_model_set_persistent_decode(self.h, int(on)), "set_persistent_decode")

    def close(self) -> None:
        if getattr(self, "h", None):
            host().axon_model_free(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def new_cache(self) -> int:
        c = C.c_int(-1)
        _mcheck(host().axon_model_cache_new(self.h, C.byref(c)), "cache_new")
        return c.value

    def free_cache(self, cache: int) -> None:
        _mcheck(host().axon_model_cache_free(self.h, cache), "cache_free")

    def cache_pos(self, cache: int) -> int:
        p = C.c_size_t(0)
        _mcheck(host().axon_model_cache_pos(self.h, cache, C.byref(p)), "cache_pos")
        return p.value

    def truncate(self, cache: int, pos: int) -> None:
        _mcheck(host().axon_model_cache_truncate(self.h, cache, pos), "cache_truncate")

    def cache_rows(self, cache: int, layer: int, values: bool, n: int) -> np.ndarray:
        out = np.zeros((n, self.info.n_head_kv * self.info.head_dim), np.float32)
        _mcheck(host().axon_model_cache_read(self.h, cache, layer, int(values), n, out.ctypes.data), "cache_read")
        return out

    def cache_fill(self, cache: int, rows) -> None:
        """Positions [pos, pos + n) of every layer's K and V from rows [n_layer][2][n][n_kv * head_dim]
        (float32), as if prefilled (axon_model_cache_fill)."""
        r = np.ascontiguousarray(rows, np.float32)
        row = self.info.n_head_kv * self.info.head_dim
        if r.ndim != 4 or r.shape[0] != self.info.n_layer or r.shape[1] != 2 or r.shape[3] != row:
            raise ValueError(f"cache_fill: rows of shape {r.shape}, expected [n_layer][2][n][{row}]")
        _mcheck(host().axon_model_cache_fill(self.h, cache, r.ctypes.data, r.shape[2]), "cache_fill")

    def _logits(self, n: int, want: bool):
        return np.zeros((n, self.n_vocab), np.float32) if want else None

    def forward(self, tokens, logits: bool = True):
        t = np.ascontiguousarray(tokens, np.int32)
        out = self._logits(len(t), logits)
        _mcheck(host().axon_model_forward(self.h, t.ctypes.data, len(t),
                                         out.ctypes.data if out is not None else None), "forward")
        return out

    def forward_prefill(self, cache: int, tokens, logits: bool = True):
        t = np.ascontiguousarray(tokens, np.int32)
        out = self._logits(len(t), logits)
        _mcheck(host().axon_model_forward_prefill(self.h, cache, t.ctypes.data, len(t),
                                                 out.ctypes.data if out is not None else None), "forward_prefill")
        return out

    def forward_batch(self, caches, tokens, logits: bool = True):
        t = np.ascontiguousarray(tokens, np.int32)
        cs = np.ascontiguousarray(caches, np.int32)
        out = self._logits(len(t), logits)
        _mcheck(host().axon_model_forward_batch(self.h, cs.ctypes.data, t.ctypes.data, len(t),
                                               out.ctypes.data if out is not None else None), "forward_batch")
        return out

    def forward_mixed(self, prefill_cache, chunk, caches, tokens, logits: bool = True):
        """One continuous-batching step as one pass (axon_model_forward_mixed): `chunk` into
        prefill_cache (None with an empty chunk), tokens[i] into caches[i]. Returns the chunk's
        last row of logits (if any) then one row per decode cache."""
        ch = np.ascontiguousarray(chunk if chunk is not None else [], np.int32)
        t = np.ascontiguousarray(tokens, np.int32)
        cs = np.ascontiguousarray(caches, np.int32)
        if len(cs) != len(t):
            raise ValueError(f"forward_mixed: {len(cs)} caches for {len(t)} tokens")
        out = self._logits(int(len(ch) > 0) + len(t), logits)
        _mcheck(host().axon_model_forward_mixed(self.h, -1 if prefill_cache is None else prefill_cache,
                                               ch.ctypes.data if len(ch) else None, len(ch),
                                               cs.ctypes.data if len(cs) else None, t.ctypes.data if len(t) else None,
                                               len(t), out.ctypes.data if out is not None else None), "forward_mixed")
        return out

    def generate_greedy(self, cache: int, token: int, n: int) -> np.ndarray:
        """n greedy steps after `token` with the ids kept on the device between steps
        (axon_model_generate_greedy); the n chosen ids."""
        out = np.zeros(n, np.int32)
        _mcheck(host().axon_model_generate_greedy(self.h, cache, int(token), n, out.ctypes.data), "generate_greedy")
        return out

    def greedy(self, n: int, recent=None, repeat_penalty: float = 1.0, repeat_last_n: int = 64) -> np.ndarray:
        """Sampler::sample at temperature zero over the last pass's n rows, on the device
        (src/sampling/sampler.cpp:67-102): the repetition penalty over recent[i], row i's token
        history, then the first maximum. Consumes the pass's logits."""
        ids = np.empty(n, np.int32)
        rec = lens = None
        if recent is not None:
            arrs = [np.ascontiguousarray(r, np.int32) for r in recent]
            rec = (C.c_void_p * n)(*[a.ctypes.data if len(a) else None for a in arrs])
            lens = (C.c_size_t * n)(*[len(a) for a in arrs])
        _mcheck(host().axon_model_greedy(self.h, rec, lens, repeat_penalty, repeat_last_n, ids.ctypes.data, n),
                "greedy")
        return ids

    def sample(self, configs, rngs, recent=None) -> np.ndarray:
        """Sampler::sample over the last pass's rows (axon_model_sample): row i with configs[i]
        and rngs[i] (advanced by one draw when its temperature is above zero)."""
        n = len(configs)
        if len(rngs) != n:
            raise ValueError(f"sample: {len(rngs)} generators for {n} configs")
        cfg = (SamplerConfig * n)(*configs)
        rs = (Rng * n)()
        for i, r in enumerate(rngs):
            C.memmove(C.byref(rs[i]), C.byref(r), C.sizeof(Rng))
        ids = np.empty(n, np.int32)
        rec = lens = None
        if recent is not None:
            arrs = [np.ascontiguousarray(r, np.int32) for r in recent]
            rec = (C.c_void_p * n)(*[a.ctypes.data if len(a) else None for a in arrs])
            lens = (C.c_size_t * n)(*[len(a) for a in arrs])
        _mcheck(host().axon_model_sample(self.h, cfg, rs, rec, lens, ids.ctypes.data, n), "sample")
        for i, r in enumerate(rngs):
            C.memmove(C.byref(r), C.byref(rs[i]), C.sizeof(Rng))
        return ids

    def probe(self, weight_type: int, enable: bool = True) -> None:
        _mcheck(host().axon_model_probe(self.h, weight_type, int(enable)), "probe")

    def probe_read(self):
        """(device ms, launches, algorithmic bytes) of the probed launches since the last read."""
        ms, n, b = C.c_double(0), C.c_size_t(0), C.c_double(0)
        _mcheck(host().axon_model_probe_read(self.h, C.byref(ms), C.byref(n), C.byref(b)), "probe_read")
        return ms.value, n.value, b.value
