"""Test-side helpers: block dtypes, the .axt fixture reader, a GGUF v3 reader, and ctypes
bindings for the CPU oracle (oracle/liboracle.so) and the reference build
(oracle/_ref/libaxonref.so). Only tests, smoke() and bench.py's cpu_baseline use these."""
from __future__ import annotations

import ctypes as C
import os
import struct
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
GOLDEN = ROOT / "tests" / "golden"
ORACLE_SO = ROOT / "oracle" / "liboracle.so"
REF_SO = ROOT / "oracle" / "_ref" / "libaxonref.so"

# Block layouts of src/core/dtype.h:85-120 as packed numpy records.
Q8_0 = np.dtype([("d", "<u2"), ("qs", "i1", 32)])
Q4_0 = np.dtype([("d", "<u2"), ("qs", "u1", 16)])
Q4_1 = np.dtype([("d", "<u2"), ("m", "<u2"), ("qs", "u1", 16)])
Q6_K = np.dtype([("ql", "u1", 128), ("qh", "u1", 64), ("scales", "i1", 16), ("d", "<u2")])
assert (Q8_0.itemsize, Q4_0.itemsize, Q4_1.itemsize, Q6_K.itemsize) == (34, 18, 20, 210)

F32, F16, Q4_0_ID, Q4_1_ID, Q8_0_ID, Q6_K_ID, BF16 = 0, 1, 2, 3, 8, 14, 30
BLOCK = {Q8_0_ID: (32, Q8_0), Q4_0_ID: (32, Q4_0), Q4_1_ID: (32, Q4_1), Q6_K_ID: (256, Q6_K)}


def row_bytes(type_id: int, n: int) -> int:
    if type_id == F32:
        return 4 * n
    if type_id in (F16, BF16):
        return 2 * n
    qk, dt = BLOCK[type_id]
    return n // qk * dt.itemsize


# ---------------------------------------------------------------------------------------------
# .axt fixtures (src/core/axt.h:3): "AXT1", u32 ndim, u64 dims, u32 dtype, raw data.

def read_axt(path: Path) -> np.ndarray:
    raw = Path(path).read_bytes()
    assert raw[:4] == b"AXT1", path
    ndim = struct.unpack_from("<I", raw, 4)[0]
    dims = struct.unpack_from("<" + "Q" * ndim, raw, 8)
    off = 8 + 8 * ndim
    dtype = struct.unpack_from("<I", raw, off)[0]
    off += 4
    np_t = {0: "<f4", 1: "<u2", 2: "<u2", 3: "<i4"}[dtype]
    return np.frombuffer(raw, dtype=np_t, offset=off).reshape(dims).copy()


def golden(name: str) -> np.ndarray:
    return read_axt(GOLDEN / name)


def golden_blocks(name: str, dt: np.dtype) -> np.ndarray:
    return np.frombuffer((GOLDEN / name).read_bytes(), dtype=dt).copy()


# ---------------------------------------------------------------------------------------------
# GGUF v3 reader (the subset of src/core/gguf.cpp:484-662 the tests need).

_SCALAR = {0: "B", 1: "b", 2: "H", 3: "h", 4: "I", 5: "i", 6: "f", 7: "?", 10: "Q", 11: "q", 12: "d"}


class GGUF:
    def __init__(self, path: Path):
        self.path = Path(path)
        self.buf = np.memmap(self.path, dtype=np.uint8, mode="r")
        mv = memoryview(self.buf)
        self._off = 0

        def rd(fmt):
            v = struct.unpack_from("<" + fmt, mv, self._off)
            self._off += struct.calcsize("<" + fmt)
            return v[0]

        def rs():
            n = rd("Q")
            s = bytes(mv[self._off:self._off + n]).decode("utf-8", "replace")
            self._off += n
            return s

        def rv(t):
            if t in _SCALAR:
                return rd(_SCALAR[t])
            if t == 8:
                return rs()
            if t == 9:
                et, n = rd("I"), rd("Q")
                return [rv(et) for _ in range(n)]
            raise ValueError(f"gguf value type {t}")

        assert rd("I") == 0x46554747, "gguf magic"
        assert rd("I") == 3, "gguf version"
        n_t, n_kv = rd("Q"), rd("Q")
        self.meta = {}
        for _ in range(n_kv):
            k = rs()
            self.meta[k] = rv(rd("I"))
        self.tensors = {}
        for _ in range(n_t):
            name = rs()
            nd = rd("I")
            dims = [rd("Q") for _ in range(nd)]
            self.tensors[name] = (dims, rd("I"), rd("Q"))
        align = self.meta.get("general.alignment", 32)
        self.data_offset = (self._off + align - 1) // align * align

    def tensor_bytes(self, name: str) -> np.ndarray:
        dims, t, off = self.tensors[name]
        rows = int(np.prod(dims[1:])) if len(dims) > 1 else 1
        n = row_bytes(t, dims[0]) * rows
        start = self.data_offset + off
        return self.buf[start:start + n]

    def tensor_info(self, name: str):
        return self.tensors.get(name)


# ---------------------------------------------------------------------------------------------
# ctypes plumbing

def ptr(a: np.ndarray) -> C.c_void_p:
    return C.c_void_p(a.ctypes.data) if a is not None else C.c_void_p(0)


def _load(path: Path) -> C.CDLL | None:
    if not path.exists():
        return None
    return C.CDLL(str(path))


_oracle = None


def oracle() -> C.CDLL:
    global _oracle
    if _oracle is None:
        lib = _load(ORACLE_SO)
        assert lib is not None, f"{ORACLE_SO} missing: run __graft_entry__.build()"
        lib.ora_fp16_to_fp32.restype = C.c_float
        lib.ora_fp16_to_fp32.argtypes = [C.c_uint16]
        lib.ora_fp32_to_fp16.restype = C.c_uint16
        lib.ora_fp32_to_fp16.argtypes = [C.c_float]
        lib.ora_bf16_to_fp32.restype = C.c_float
        lib.ora_bf16_to_fp32.argtypes = [C.c_uint16]
        lib.ora_fp32_to_bf16.restype = C.c_uint16
        lib.ora_fp32_to_bf16.argtypes = [C.c_float]
        lib.ora_workspace_floats.restype = C.c_size_t
        lib.ora_rng_next.restype = C.c_uint64
        lib.ora_rng_uniform.restype = C.c_double
        lib.ora_sample.restype = C.c_int32
        _oracle = lib
    return _oracle


_ref = None


def ref() -> C.CDLL | None:
    """The reference's own scalar table and LlamaModel, or None when oracle/_ref was not built."""
    global _ref
    if _ref is None:
        lib = _load(REF_SO)
        if lib is None:
            return None
        lib.ref_fp16_to_fp32.restype = C.c_float
        lib.ref_fp16_to_fp32.argtypes = [C.c_uint16]
        lib.ref_fp32_to_fp16.restype = C.c_uint16
        lib.ref_fp32_to_fp16.argtypes = [C.c_float]
        lib.ref_model_load.restype = C.c_void_p
        lib.ref_model_load.argtypes = [C.c_char_p, C.c_size_t, C.c_size_t, C.c_size_t, C.c_int, C.c_int,
                                       C.c_char_p, C.c_size_t]
        lib.ref_model_load_cache.restype = C.c_void_p
        lib.ref_model_load_cache.argtypes = [C.c_char_p, C.c_size_t, C.c_size_t, C.c_size_t, C.c_int, C.c_int,
                                             C.c_int, C.c_char_p, C.c_size_t]
        for f in ("ref_model_free", "ref_model_threads", "ref_cache_new"):
            getattr(lib, f).argtypes = [C.c_void_p]
        lib.ref_model_weight_bytes.restype = C.c_size_t
        lib.ref_model_weight_bytes.argtypes = [C.c_void_p]
        lib.ref_cache_pos.restype = C.c_size_t
        lib.ref_cache_pos.argtypes = [C.c_void_p, C.c_int]
        lib.ref_cache_truncate.argtypes = [C.c_void_p, C.c_int, C.c_size_t]
        lib.ref_cache_fill.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_size_t]
        lib.ref_forward.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p]
        lib.ref_forward_prefill.argtypes = [C.c_void_p, C.c_int, C.c_void_p, C.c_size_t, C.c_void_p]
        lib.ref_forward_batch.argtypes = [C.c_void_p, C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p]
        _ref = lib
    return _ref


SZ = C.c_size_t
FL = C.c_float


def call(lib: C.CDLL, name: str, *args):
    """Calls name(*args) with numpy arrays passed as pointers, ints as size_t, floats as float."""
    conv = []
    for a in args:
        if isinstance(a, np.ndarray):
            conv.append(ptr(a))
        elif a is None:
            conv.append(C.c_void_p(0))
        elif isinstance(a, float):
            conv.append(FL(a))
        elif isinstance(a, (C._SimpleCData, C.c_void_p)):
            conv.append(a)
        else:
            conv.append(SZ(a))
    return getattr(lib, name)(*conv)


# ---------------------------------------------------------------------------------------------
# Oracle model structs (oracle/oracle.h)

class OraTensor(C.Structure):
    _fields_ = [("data", C.c_void_p), ("type", C.c_int), ("ne0", C.c_uint64), ("ne1", C.c_uint64)]


class OraLayer(C.Structure):
    _fields_ = [(n, OraTensor) for n in ("attn_norm", "wq", "wk", "wv", "wo", "ffn_norm", "w_gate", "w_up",
                                          "w_down", "bq", "bk", "bv")]


class OraModel(C.Structure):
    _fields_ = [("n_layer", C.c_uint32), ("n_embd", C.c_uint32), ("n_head", C.c_uint32),
                ("n_head_kv", C.c_uint32), ("n_ff", C.c_uint32), ("n_vocab", C.c_uint32),
                ("head_dim", C.c_uint32), ("rotary_dim", C.c_uint32), ("rope_theta", C.c_float),
                ("rms_eps", C.c_float), ("rope_style", C.c_int), ("exact_activations", C.c_int),
                ("token_embd", OraTensor), ("output_norm", OraTensor), ("output", OraTensor),
                ("rope_freqs", C.c_void_p), ("layers", C.POINTER(OraLayer))]


class OraCache(C.Structure):
    _fields_ = [("base", C.c_void_p), ("max_ctx", C.c_size_t), ("pos", C.c_size_t), ("f16", C.c_int)]


class ModelConfig:
    """LlamaConfig::from_gguf (src/model/config.cpp:27-123), the fields the forward needs."""

    def __init__(self, g: GGUF):
        arch = g.meta["general.architecture"]
        k = lambda s: f"{arch}.{s}"  # noqa: E731
        self.arch = arch
        self.rope_style = 0 if arch == "llama" else 1
        self.n_layer = g.meta[k("block_count")]
        self.n_embd = g.meta[k("embedding_length")]
        self.n_head = g.meta[k("attention.head_count")]
        self.n_head_kv = g.meta.get(k("attention.head_count_kv"), self.n_head)
        self.n_ff = g.meta[k("feed_forward_length")]
        self.n_ctx_train = g.meta[k("context_length")]
        self.head_dim = g.meta.get(k("attention.key_length"), self.n_embd // self.n_head)
        self.rotary_dim = g.meta.get(k("rope.dimension_count"), self.head_dim)
        self.rope_theta = float(np.float32(g.meta.get(k("rope.freq_base"), 10000.0)))
        self.rms_eps = float(np.float32(g.meta.get(k("attention.layer_norm_rms_epsilon"), 1e-5)))
        self.n_vocab = g.tensors["token_embd.weight"][0][1]
        self.tied = "output.weight" not in g.tensors
        self.bias = "blk.0.attn_q.bias" in g.tensors
        self.llama3 = "rope_freqs.weight" in g.tensors


class OracleModel:
    """The oracle's forward pass over a GGUF file's tensors (host memory, zero-copy)."""

    def __init__(self, path: Path, exact_activations: bool = False):
        self.g = GGUF(path)
        self.cfg = cfg = ModelConfig(self.g)
        self._keep = []

        def t(name):
            dims, typ, _ = self.g.tensors[name]
            data = self.g.tensor_bytes(name)
            self._keep.append(data)
            return OraTensor(data.ctypes.data, typ, dims[0], dims[1] if len(dims) > 1 else 1)

        layers = (OraLayer * cfg.n_layer)()
        for i in range(cfg.n_layer):
            p = f"blk.{i}."
            L = layers[i]
            for f, n in (("attn_norm", "attn_norm"), ("wq", "attn_q"), ("wk", "attn_k"), ("wv", "attn_v"),
                         ("wo", "attn_output"), ("ffn_norm", "ffn_norm"), ("w_gate", "ffn_gate"),
                         ("w_up", "ffn_up"), ("w_down", "ffn_down")):
                setattr(L, f, t(p + n + ".weight"))
            if cfg.bias:
                L.bq, L.bk, L.bv = t(p + "attn_q.bias"), t(p + "attn_k.bias"), t(p + "attn_v.bias")
        self.layers = layers
        m = OraModel()
        for f in ("n_layer", "n_embd", "n_head", "n_head_kv", "n_ff", "n_vocab", "head_dim", "rotary_dim",
                  "rope_theta", "rms_eps", "rope_style"):
            setattr(m, f, getattr(cfg, f))
        m.exact_activations = int(exact_activations)
        m.token_embd = t("token_embd.weight")
        m.output_norm = t("output_norm.weight")
        m.output = m.token_embd if cfg.tied else t("output.weight")
        m.rope_freqs = t("rope_freqs.weight").data if cfg.llama3 else None
        m.layers = layers
        self.m = m
        self.lib = oracle()

    def new_cache(self, max_ctx: int, f16: bool = False):
        """A cache of float elements (CacheType::F32) or fp16 bit patterns (CacheType::F16)."""
        row = self.cfg.n_head_kv * self.cfg.head_dim
        store = np.zeros(self.cfg.n_layer * 2 * max_ctx * row, dtype=np.uint16 if f16 else np.float32)
        c = OraCache(store.ctypes.data, max_ctx, 0, int(f16))
        c._store = store
        return c

    def _ws(self, n, ctx):
        n_f = self.lib.ora_workspace_floats(C.byref(self.m), SZ(n), SZ(ctx))
        return np.zeros(n_f, dtype=np.float32)

    def forward(self, tokens, cache=None) -> np.ndarray:
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        n = len(tokens)
        ctx = (cache.pos if cache is not None else 0) + n
        ws = self._ws(n, ctx)
        logits = np.zeros((n, self.cfg.n_vocab), dtype=np.float32)
        rc = self.lib.ora_forward(C.byref(self.m), ptr(tokens), SZ(n),
                                  C.byref(cache) if cache is not None else None, ptr(ws), ptr(logits))
        assert rc == 0, rc
        return logits

    def forward_batch(self, tokens, caches) -> np.ndarray:
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        n = len(tokens)
        arr = (C.POINTER(OraCache) * n)(*[C.pointer(c) for c in caches])
        ctx = max(c.pos for c in caches) + 1
        ws = self._ws(n, ctx)
        logits = np.zeros((n, self.cfg.n_vocab), dtype=np.float32)
        rc = self.lib.ora_forward_batch(C.byref(self.m), ptr(tokens), SZ(n), arr, ptr(ws), ptr(logits))
        assert rc == 0, rc
        return logits


class RefModel:
    """The reference's own LlamaModel (scalar table) through oracle/_ref."""

    def __init__(self, path: Path, max_seq=32, max_ctx=128, max_batch=1, n_threads=1, exact=False, f16=False):
        self.lib = ref()
        assert self.lib is not None
        err = C.create_string_buffer(512)
        self.h = self.lib.ref_model_load_cache(str(path).encode(), max_seq, max_ctx, max_batch, n_threads,
                                               int(exact), int(f16), err, 512)
        assert self.h, err.value.decode()
        self.n_vocab = ModelConfig(GGUF(path)).n_vocab

    def __del__(self):
        if getattr(self, "h", None):
            self.lib.ref_model_free(C.c_void_p(self.h))

    def forward(self, tokens):
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        out = np.zeros((len(tokens), self.n_vocab), dtype=np.float32)
        assert self.lib.ref_forward(C.c_void_p(self.h), ptr(tokens), len(tokens), ptr(out)) == 0
        return out

    def new_cache(self) -> int:
        return self.lib.ref_cache_new(C.c_void_p(self.h))

    def forward_prefill(self, cache: int, tokens):
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        out = np.zeros((len(tokens), self.n_vocab), dtype=np.float32)
        assert self.lib.ref_forward_prefill(C.c_void_p(self.h), cache, ptr(tokens), len(tokens), ptr(out)) == 0
        return out

    def forward_batch(self, caches, tokens):
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        ids = np.ascontiguousarray(caches, dtype=np.int32)
        out = np.zeros((len(tokens), self.n_vocab), dtype=np.float32)
        assert self.lib.ref_forward_batch(C.c_void_p(self.h), ptr(ids), ptr(tokens), len(tokens), ptr(out)) == 0
        return out


def have_ref() -> bool:
    return REF_SO.exists() and os.environ.get("AXON_NO_REF") is None
