"""Seeded random-init GGUF models and the weight quantizers that write them.

The benchmark configurations of this repository are LLaMA-family shapes with random weights
(no checkpoints are available offline): every weight ~ N(0, 0.02), norm gains ~ 1 + N(0, 0.01),
optional Qwen2 Q/K/V biases ~ N(0, 0.02), and for Llama 3 shapes the rope frequency factors of
the published llama3 scaling. Files are GGUF v3 that trickymind1324/axon-infer's reader accepts
(src/core/gguf.cpp:484-662; metadata keys of src/model/config.cpp:27-123; a minimal byte-level
"gpt2" vocabulary so src/tokenizer/vocab.cpp:19-141 loads).

Quantizers, all in float32 with numpy:
  Q8_0  the repository's quantize_row_q8_0 (src/core/dtype.cpp:338-354): d = amax / 127,
        q = roundf(x / d) with ties away from zero.
  Q4_0  ggml's reference block quantizer: d = (signed value of largest magnitude) / -8,
        q = min(15, trunc(x / d + 8.5)).
  Q4_1  ggml's reference: d = (max - min) / 15, m = min, q = min(15, trunc((x - m) / d + 0.5)).
  Q6_K  a plain absmax quantizer into the ggml super-block layout: per 16-element group a
        scale s = amax / 31, d = max|s| / 127, int8 group scales round(s / d), 6-bit
        q = clamp(round(x / (d * sc)), -32, 31) + 32. Any valid Q6_K bytes serve: the
        reference holds no Q6_K quantizer and no fixture pins one.
"""
from __future__ import annotations

import hashlib
import json
import os
import struct
from dataclasses import asdict, dataclass, field
from pathlib import Path

import numpy as np

F32, F16, Q4_0, Q4_1, Q8_0, Q6_K, BF16 = 0, 1, 2, 3, 8, 14, 30
BLOCK_BYTES = {Q8_0: (32, 34), Q4_0: (32, 18), Q4_1: (32, 20), Q6_K: (256, 210)}

Q8_0_DT = np.dtype([("d", "<u2"), ("qs", "i1", 32)])
Q4_0_DT = np.dtype([("d", "<u2"), ("qs", "u1", 16)])
Q4_1_DT = np.dtype([("d", "<u2"), ("m", "<u2"), ("qs", "u1", 16)])
Q6_K_DT = np.dtype([("ql", "u1", 128), ("qh", "u1", 64), ("scales", "i1", 16), ("d", "<u2")])


# ---------------------------------------------------------------------------------------------
# Quantizers (x: float32 array whose length is a whole number of blocks)

def _roundf(v: np.ndarray) -> np.ndarray:
    """C roundf: nearest, ties away from zero, exact in float32."""
    t = np.trunc(v)
    frac = np.abs(v - t)
    return t + np.where(frac >= np.float32(0.5), np.sign(v), np.float32(0)).astype(np.float32)


def _fp16_bits(v: np.ndarray) -> np.ndarray:
    return np.asarray(v, np.float32).astype(np.float16).view(np.uint16)


def quantize_q8_0(x: np.ndarray) -> np.ndarray:
    b = np.asarray(x, np.float32).reshape(-1, 32)
    amax = np.max(np.abs(b), axis=1)
    d = (amax / np.float32(127)).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(d != 0, np.float32(1) / np.where(d != 0, d, np.float32(1)), np.float32(0)).astype(np.float32)
    q = _roundf((b * inv[:, None]).astype(np.float32))
    out = np.empty(b.shape[0], Q8_0_DT)
    out["d"] = _fp16_bits(d)
    out["qs"] = q.astype(np.int8)
    return out


def quantize_q4_0(x: np.ndarray) -> np.ndarray:
    b = np.asarray(x, np.float32).reshape(-1, 32)
    idx = np.argmax(np.abs(b), axis=1)
    mx = b[np.arange(b.shape[0]), idx]
    d = (mx / np.float32(-8)).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(d != 0, np.float32(1) / np.where(d != 0, d, np.float32(1)), np.float32(0)).astype(np.float32)
    v = (b * inv[:, None]).astype(np.float32) + np.float32(8.5)
    q = np.minimum(15, np.trunc(v).astype(np.int32)).astype(np.uint8)
    out = np.empty(b.shape[0], Q4_0_DT)
    out["d"] = _fp16_bits(d)
    out["qs"] = q[:, :16] | (q[:, 16:] << 4)
    return out


def quantize_q4_1(x: np.ndarray) -> np.ndarray:
    b = np.asarray(x, np.float32).reshape(-1, 32)
    lo = np.min(b, axis=1)
    hi = np.max(b, axis=1)
    d = ((hi - lo) / np.float32(15)).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(d != 0, np.float32(1) / np.where(d != 0, d, np.float32(1)), np.float32(0)).astype(np.float32)
    v = ((b - lo[:, None]) * inv[:, None]).astype(np.float32) + np.float32(0.5)
    q = np.minimum(15, np.trunc(v).astype(np.int32)).astype(np.uint8)
    out = np.empty(b.shape[0], Q4_1_DT)
    out["d"] = _fp16_bits(d)
    out["m"] = _fp16_bits(lo)
    out["qs"] = q[:, :16] | (q[:, 16:] << 4)
    return out


def quantize_q6_k(x: np.ndarray) -> np.ndarray:
    b = np.asarray(x, np.float32).reshape(-1, 16, 16)   # super-block, group, element
    nsb = b.shape[0]
    s = np.max(np.abs(b), axis=2) / np.float32(31)      # group scales [nsb][16]
    dmax = np.max(np.abs(s), axis=1) / np.float32(127)
    d16 = _fp16_bits(dmax)
    d = d16.view(np.float16).astype(np.float32)
    with np.errstate(divide="ignore", invalid="ignore"):
        sc = np.where(d[:, None] > 0, np.rint(s / np.where(d[:, None] > 0, d[:, None], 1)), 0)
    sc = np.clip(sc, -128, 127).astype(np.int8)
    step = (d[:, None] * sc.astype(np.float32)).astype(np.float32)  # [nsb][16]
    with np.errstate(divide="ignore", invalid="ignore"):
        q = np.where(step[:, :, None] != 0, np.rint(b / np.where(step[:, :, None] != 0, step[:, :, None], 1)), 0)
    q = (np.clip(q, -32, 31) + 32).astype(np.uint8).reshape(nsb, 256)
    # ggml layout: for each 128-half n and l in 0..31, y[l], y[l+32], y[l+64], y[l+96]
    # come from ql[l] low, ql[l+32] low, ql[l] high, ql[l+32] high with 2 high bits each in qh[l].
    out = np.zeros(nsb, Q6_K_DT)
    ql = np.zeros((nsb, 128), np.uint8)
    qh = np.zeros((nsb, 64), np.uint8)
    for n in range(2):
        y = q[:, n * 128:(n + 1) * 128]
        q1, q2, q3, q4 = y[:, 0:32], y[:, 32:64], y[:, 64:96], y[:, 96:128]
        ql[:, n * 64:n * 64 + 32] = (q1 & 0x0F) | ((q3 & 0x0F) << 4)
        ql[:, n * 64 + 32:n * 64 + 64] = (q2 & 0x0F) | ((q4 & 0x0F) << 4)
        qh[:, n * 32:n * 32 + 32] = (q1 >> 4) | ((q2 >> 4) << 2) | ((q3 >> 4) << 4) | ((q4 >> 4) << 6)
    out["ql"] = ql
    out["qh"] = qh
    out["scales"] = sc
    out["d"] = d16
    return out


QUANTIZERS = {Q8_0: quantize_q8_0, Q4_0: quantize_q4_0, Q4_1: quantize_q4_1, Q6_K: quantize_q6_k}


def tensor_bytes(type_id: int, values: np.ndarray) -> bytes:
    if type_id == F32:
        return np.asarray(values, np.float32).tobytes()
    if type_id == F16:
        return _fp16_bits(values).tobytes()
    return QUANTIZERS[type_id](values).tobytes()


def row_bytes(type_id: int, n: int) -> int:
    if type_id == F32:
        return 4 * n
    if type_id in (F16, BF16):
        return 2 * n
    qk, bs = BLOCK_BYTES[type_id]
    assert n % qk == 0, (type_id, n)
    return n // qk * bs


# ---------------------------------------------------------------------------------------------
# GGUF v3 writer

_GGUF_TYPES = {"u32": 4, "i32": 5, "f32": 6, "bool": 7, "str": 8, "arr": 9, "u64": 10}


def _kv(key: str, kind: str, value) -> bytes:
    out = struct.pack("<Q", len(key.encode())) + key.encode()
    if kind == "str":
        v = value.encode()
        return out + struct.pack("<IQ", 8, len(v)) + v
    if kind == "u32":
        return out + struct.pack("<II", 4, value)
    if kind == "i32":
        return out + struct.pack("<Ii", 5, value)
    if kind == "f32":
        return out + struct.pack("<If", 6, value)
    if kind == "bool":
        return out + struct.pack("<IB", 7, 1 if value else 0)
    if kind == "str_arr":
        body = b"".join(struct.pack("<Q", len(s.encode())) + s.encode() for s in value)
        return out + struct.pack("<IIQ", 9, 8, len(value)) + body
    if kind == "i32_arr":
        return out + struct.pack("<IIQ", 9, 5, len(value)) + np.asarray(value, np.int32).tobytes()
    raise ValueError(kind)


def _gpt2_byte_chars() -> list[str]:
    """The printable stand-ins GPT-2's byte-level BPE uses for the 256 byte values."""
    keep = list(range(ord("!"), ord("~") + 1)) + list(range(0xA1, 0xAC + 1)) + list(range(0xAE, 0xFF + 1))
    chars = {b: chr(b) for b in keep}
    n = 0
    for b in range(256):
        if b not in chars:
            chars[b] = chr(256 + n)
            n += 1
    return [chars[b] for b in range(256)]


def write_gguf(path: Path, metadata: list, tensors: list) -> None:
    """metadata: [(key, kind, value)]; tensors: [(name, type_id, dims (innermost first), writer)]
    where writer(f) writes exactly the tensor's bytes. Alignment 32."""
    align = 32
    head = struct.pack("<IIQQ", 0x46554747, 3, len(tensors), len(metadata))
    head += b"".join(_kv(k, kind, v) for k, kind, v in metadata)
    infos = b""
    offset = 0
    sizes = []
    for name, type_id, dims, _ in tensors:
        rows = int(np.prod(dims[1:])) if len(dims) > 1 else 1
        nbytes = row_bytes(type_id, dims[0]) * rows
        infos += struct.pack("<Q", len(name.encode())) + name.encode() + struct.pack("<I", len(dims))
        infos += struct.pack(f"<{len(dims)}Q", *dims) + struct.pack("<IQ", type_id, offset)
        sizes.append(nbytes)
        offset = (offset + nbytes + align - 1) // align * align
    blob = head + infos
    pad = (-len(blob)) % align
    tmp = Path(str(path) + ".tmp")
    with open(tmp, "wb") as f:
        f.write(blob + b"\0" * pad)
        for (name, type_id, dims, writer), nbytes in zip(tensors, sizes):
            start = f.tell()
            writer(f)
            assert f.tell() - start == nbytes, (name, f.tell() - start, nbytes)
            f.write(b"\0" * ((-nbytes) % align))
    os.replace(tmp, path)


# ---------------------------------------------------------------------------------------------
# Model shapes

@dataclass
class ModelSpec:
    name: str
    arch: str = "llama"
    n_embd: int = 576
    n_layer: int = 30
    n_head: int = 9
    n_head_kv: int = 3
    n_ff: int = 1536
    n_vocab: int = 49152
    n_ctx: int = 8192
    rope_theta: float = 100000.0
    rms_eps: float = 1e-5
    tied: bool = True
    bias: bool = False
    llama3: bool = False
    wtype: int = Q8_0                   # attention and feed-forward weights
    q4_1_tensors: tuple = ()           # names (per layer suffix) stored as Q4_1 instead
    out_type: int = Q8_0                # output matrix (or tied embedding)
    embd_type: int | None = None        # embedding when untied (None: wtype)
    seed: int = 0

    def key(self) -> str:
        blob = json.dumps(asdict(self), sort_keys=True).encode()
        return hashlib.sha256(blob).hexdigest()[:16]


# The BASELINE configurations (C1, C3, C4, C5); C2 is a kernel sweep, not a model.
SMOLLM2_135M = ModelSpec("smollm2-135m", n_embd=576, n_layer=30, n_head=9, n_head_kv=3, n_ff=1536, n_vocab=49152,
                         rope_theta=100000.0, tied=True, wtype=Q8_0, out_type=Q8_0)
TINYLLAMA_1B = ModelSpec("tinyllama-1.1b", n_embd=2048, n_layer=22, n_head=32, n_head_kv=4, n_ff=5632, n_vocab=32000,
                         n_ctx=2048, rope_theta=10000.0, tied=False, wtype=Q4_0,
                         q4_1_tensors=("ffn_down",), out_type=Q6_K, embd_type=Q4_0)
LLAMA32_1B = ModelSpec("llama-3.2-1b", n_embd=2048, n_layer=16, n_head=32, n_head_kv=8, n_ff=8192, n_vocab=128256,
                       n_ctx=131072, rope_theta=500000.0, tied=True, llama3=True, wtype=Q4_0, out_type=Q6_K)
QWEN25_05B = ModelSpec("qwen2.5-0.5b", arch="qwen2", n_embd=896, n_layer=24, n_head=14, n_head_kv=2, n_ff=4864,
                       n_vocab=151936, n_ctx=32768, rope_theta=1000000.0, tied=False, bias=True, wtype=Q4_0,
                       out_type=Q8_0, embd_type=Q4_0, rms_eps=1e-6)
CONFIGS = {"c1": SMOLLM2_135M, "c3": TINYLLAMA_1B, "c4": LLAMA32_1B, "c5": QWEN25_05B}


def llama3_factors(rotary_dim: int, theta: float, factor=32.0, low=1.0, high=4.0, orig_ctx=8192) -> np.ndarray:
    """Llama 3.1/3.2 rope frequency divisors (the published scaling rule), as GGUF converters
    store them in rope_freqs.weight."""
    inv = theta ** (-np.arange(0, rotary_dim, 2, dtype=np.float64) / rotary_dim)
    wavelen = 2 * np.pi / inv
    low_wl, high_wl = orig_ctx / low, orig_ctx / high
    out = np.ones_like(inv)
    out[wavelen > low_wl] = factor
    mid = (wavelen <= low_wl) & (wavelen >= high_wl)
    smooth = (orig_ctx / wavelen[mid] - low) / (high - low)
    out[mid] = 1.0 / ((1 - smooth) / factor + smooth)
    return out.astype(np.float32)


def write_model(spec: ModelSpec, path: Path, chunk_rows: int = 4096) -> Path:
    """Writes spec as a GGUF file at path (atomic). Deterministic in spec (seed included)."""
    a = spec.arch
    hd = spec.n_embd // spec.n_head
    dq, dkv = spec.n_head * hd, spec.n_head_kv * hd
    byte_chars = _gpt2_byte_chars()
    tokens = byte_chars + ["<s>", "</s>"] + [f"<t{i}>" for i in range(258, spec.n_vocab)]
    tokens = tokens[: spec.n_vocab]
    meta = [("general.architecture", "str", a), ("general.name", "str", f"axon synthetic {spec.name}"),
            (f"{a}.context_length", "u32", spec.n_ctx), (f"{a}.embedding_length", "u32", spec.n_embd),
            (f"{a}.block_count", "u32", spec.n_layer), (f"{a}.feed_forward_length", "u32", spec.n_ff),
            (f"{a}.attention.head_count", "u32", spec.n_head), (f"{a}.attention.head_count_kv", "u32", spec.n_head_kv),
            (f"{a}.rope.dimension_count", "u32", hd), (f"{a}.rope.freq_base", "f32", spec.rope_theta),
            (f"{a}.attention.layer_norm_rms_epsilon", "f32", spec.rms_eps), (f"{a}.vocab_size", "u32", spec.n_vocab),
            ("tokenizer.ggml.model", "str", "gpt2"), ("tokenizer.ggml.pre", "str", "default"),
            ("tokenizer.ggml.tokens", "str_arr", tokens), ("tokenizer.ggml.token_type", "i32_arr", [1] * len(tokens)),
            ("tokenizer.ggml.bos_token_id", "u32", 256), ("tokenizer.ggml.eos_token_id", "u32", 257),
            ("tokenizer.ggml.add_bos_token", "bool", False)]

    counter = [0]

    def gaussian(n_in: int, n_out: int, type_id: int, std=0.02, mean=0.0):
        """A writer streaming N(mean, std) rows in chunks, quantized as type_id."""
        seq = np.random.SeedSequence([spec.seed, 0xA507, counter[0]])
        counter[0] += 1

        def w(f):
            rng = np.random.default_rng(seq)
            for r0 in range(0, n_out, chunk_rows):
                r = min(chunk_rows, n_out - r0)
                vals = rng.standard_normal(r * n_in, dtype=np.float32) * np.float32(std) + np.float32(mean)
                f.write(tensor_bytes(type_id, vals))
        return w

    tensors = []
    embd_type = spec.out_type if spec.tied else (spec.embd_type if spec.embd_type is not None else spec.wtype)
    tensors.append(("token_embd.weight", embd_type, [spec.n_embd, spec.n_vocab], gaussian(spec.n_embd, spec.n_vocab, embd_type)))
    tensors.append(("output_norm.weight", F32, [spec.n_embd], gaussian(spec.n_embd, 1, F32, 0.01, 1.0)))
    if not spec.tied:
        tensors.append(("output.weight", spec.out_type, [spec.n_embd, spec.n_vocab],
                        gaussian(spec.n_embd, spec.n_vocab, spec.out_type)))
    if spec.llama3:
        fac = llama3_factors(hd, spec.rope_theta)
        tensors.append(("rope_freqs.weight", F32, [hd // 2], lambda f, fac=fac: f.write(fac.tobytes())))
    for l in range(spec.n_layer):
        p = f"blk.{l}."

        def t(suffix):
            return Q4_1 if suffix in spec.q4_1_tensors else spec.wtype
        tensors.append((p + "attn_norm.weight", F32, [spec.n_embd], gaussian(spec.n_embd, 1, F32, 0.01, 1.0)))
        for suffix, n_in, n_out in (("attn_q", spec.n_embd, dq), ("attn_k", spec.n_embd, dkv),
                                    ("attn_v", spec.n_embd, dkv), ("attn_output", dq, spec.n_embd)):
            tensors.append((p + suffix + ".weight", t(suffix), [n_in, n_out], gaussian(n_in, n_out, t(suffix))))
        if spec.bias:
            for suffix, n in (("attn_q", dq), ("attn_k", dkv), ("attn_v", dkv)):
                tensors.append((p + suffix + ".bias", F32, [n], gaussian(n, 1, F32)))
        tensors.append((p + "ffn_norm.weight", F32, [spec.n_embd], gaussian(spec.n_embd, 1, F32, 0.01, 1.0)))
        for suffix, n_in, n_out in (("ffn_gate", spec.n_embd, spec.n_ff), ("ffn_up", spec.n_embd, spec.n_ff),
                                    ("ffn_down", spec.n_ff, spec.n_embd)):
            tensors.append((p + suffix + ".weight", t(suffix), [n_in, n_out], gaussian(n_in, n_out, t(suffix))))
    path = Path(path)
    path.parent.mkdir(parents=True, exist_ok=True)
    write_gguf(path, meta, tensors)
    return path


def cached_model(spec: ModelSpec, directory: str | os.PathLike | None = None) -> Path:
    """The model file for spec under directory (default $AXON_MODEL_DIR or /tmp/axon-models),
    written on first use."""
    d = Path(directory or os.environ.get("AXON_MODEL_DIR", "/tmp/axon-models"))
    path = d / f"{spec.name}-{spec.key()}.gguf"
    if not path.exists():
        write_model(spec, path)
    return path
