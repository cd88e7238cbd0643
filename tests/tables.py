"""A common Python face for a kernel table, so one test body can run against the oracle
(C restatement), the reference build (oracle/_ref) or the HIP table. Every method takes and
returns host numpy arrays with the reference's argument meaning (src/kernels/kernels.h:33-128)."""
from __future__ import annotations

import ctypes as C

import numpy as np

from helpers import BLOCK, Q8_0, call, oracle, ref

QUANT_TYPES = ("q8_0", "q4_0", "q4_1")


class CTable:
    """The oracle (prefix "ora_") or the reference build (prefix "ref_")."""

    def __init__(self, which: str):
        self.name = which
        self.lib = oracle() if which == "oracle" else ref()
        self.p = "ora_" if which == "oracle" else "ref_"

    def _c(self, fn, *args):
        return call(self.lib, self.p + fn, *args)

    def quantize_row_q8_0(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.zeros(x.size // 32, dtype=Q8_0)
        self._c("quantize_row_q8_0", x, out, x.size)
        return out

    def matmul(self, kind: str, w, x, n_out, n_in, n_rows=None, y_stride=None):
        """kind: f32, f16, bf16, q8_0, q4_0, q4_1, q6_k (float activations) or q8_0_q8, q4_0_q8,
        q4_1_q8 (x given as Q8_0 blocks). n_rows None is the single-row entry."""
        x = np.ascontiguousarray(x)
        if n_rows is None:
            y = np.zeros(n_out, dtype=np.float32)
            self._c(f"matmul_{kind}", w, x, y, n_out, n_in)
            return y
        stride = y_stride if y_stride is not None else n_out
        y = np.full(n_rows * stride, np.float32(-7.25), dtype=np.float32)
        self._c(f"matmul_{kind}_rows", w, x, y, n_rows, n_out, n_in, stride)
        return y

    def rmsnorm(self, x, w, eps):
        y = np.zeros_like(x, dtype=np.float32)
        self._c("rmsnorm", np.ascontiguousarray(x, np.float32), np.ascontiguousarray(w, np.float32), y, x.size,
                float(eps))
        return y

    def rope(self, x, n_heads, pos, head_dim, rotary_dim, theta, style, factors=None):
        y = np.array(x, dtype=np.float32, copy=True)
        self._c("rope", y, n_heads, pos, head_dim, rotary_dim, float(theta), C.c_int(style),
                None if factors is None else np.ascontiguousarray(factors, np.float32))
        return y

    def softmax(self, x):
        y = np.array(x, dtype=np.float32, copy=True)
        self._c("softmax", y, y.size)
        return y

    def silu_mul(self, g, u):
        out = np.zeros_like(g, dtype=np.float32)
        self._c("silu_mul", np.ascontiguousarray(g, np.float32), np.ascontiguousarray(u, np.float32), out, g.size)
        return out

    def embedding_row(self, type_id, table, n, index):
        out = np.zeros(n, dtype=np.float32)
        self._c("embedding_row", C.c_int(type_id), np.ascontiguousarray(table), n, C.c_int64(index), out)
        return out

    def attention_kv_heads(self, q, k, v, n_q, n_past, n_head, n_head_kv, head_dim, scale, hb, he, f16=False):
        out = np.zeros((n_q, n_head, head_dim), dtype=np.float32)
        scores = np.zeros(n_q * (n_past + n_q), dtype=np.float32)
        self._c("attention_kv_heads_f16" if f16 else "attention_kv_heads", np.ascontiguousarray(q),
                np.ascontiguousarray(k), np.ascontiguousarray(v), out, scores, n_q, n_past, n_head, n_head_kv,
                head_dim, float(scale), hb, he)
        return out


# ------------------------------------------------------------------------------------------
# Random inputs shaped like the reference's cross-table tests (tests/unit/test_kernels_neon.cpp)

def random_floats(n, seed, scale=1.0):
    return np.random.default_rng(seed).uniform(-scale, scale, n).astype(np.float32)


def random_weights(kind: str, n_out: int, n_in: int, seed: int) -> np.ndarray:
    """Weights as the reference's tests build them: Q8_0 through the quantizer, nibble formats
    with random bytes and fixed scales (test_kernels_neon.cpp:130-146), Q6_K random super-blocks
    with a small scale (test_kernels_neon.cpp:186-200)."""
    rng = np.random.default_rng(seed)
    t = {"q8_0": 8, "q4_0": 2, "q4_1": 3, "q6_k": 14}[kind]
    qk, dt = BLOCK[t]
    nb = n_out * n_in // qk
    if kind == "q8_0":
        w = rng.uniform(-0.5, 0.5, n_out * n_in).astype(np.float32)
        return CTable("oracle").quantize_row_q8_0(w)
    b = np.zeros(nb, dtype=dt)
    if kind == "q4_0":
        b["d"] = np.float16(0.02).view(np.uint16)
        b["qs"] = rng.integers(0, 256, (nb, 16), dtype=np.uint8)
    elif kind == "q4_1":
        b["d"] = np.float16(0.02).view(np.uint16)
        b["m"] = np.float16(-0.17).view(np.uint16)
        b["qs"] = rng.integers(0, 256, (nb, 16), dtype=np.uint8)
    else:
        b["ql"] = rng.integers(0, 256, (nb, 128), dtype=np.uint8)
        b["qh"] = rng.integers(0, 256, (nb, 64), dtype=np.uint8)
        b["scales"] = rng.integers(-128, 128, (nb, 16), dtype=np.int8)
        b["d"] = np.float16(1e-3).view(np.uint16)
    return b


def dequantize(kind: str, w: np.ndarray, n_out: int, n_in: int) -> np.ndarray:
    """Dequantized weights through the oracle, for error scales."""
    t = {"q8_0": 8, "q4_0": 2, "q4_1": 3, "q6_k": 14}[kind]
    o = CTable("oracle")
    out = np.zeros((n_out, n_in), dtype=np.float32)
    for r in range(n_out):
        out[r] = o.embedding_row(t, w, n_in, r)
    return out


def relative_error(a, b, w, x):
    """|a - b| relative to sum |w_i x_i| per output (test_kernels_neon.cpp:45-59)."""
    mag = np.abs(w.astype(np.float64)) @ np.abs(x.astype(np.float64))
    return float(np.max(np.abs(a.astype(np.float64) - b.astype(np.float64)) / (mag + 1e-30)))


# ------------------------------------------------------------------------------------------
# The hip table through its C ABI (libaxon_hip.so). Same methods as CTable: host arrays in,
# host arrays out; the data crosses to HBM, the entry runs there, the result comes back.

class HipTable:
    name = "hip"

    def __init__(self):
        import axon_hip as H
        self.H = H
        H.init(0)

    def _dev(self, a):
        return self.H.DeviceBuffer.of(np.ascontiguousarray(a))

    def quantize_row_q8_0(self, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        dx = self._dev(x)
        out = self.H.DeviceBuffer(x.size // 32 * 34)
        self.H.call("quantize_row_q8_0", dx, out, x.size)
        return out.download(Q8_0)

    def matmul(self, kind: str, w, x, n_out, n_in, n_rows=None, y_stride=None):
        dw, dx = self._dev(w), self._dev(x)
        if n_rows is None:
            y = self.H.DeviceBuffer(n_out * 4)
            self.H.call(f"matmul_{kind}", dw, dx, y, n_out, n_in)
            return y.download(np.float32)
        stride = y_stride if y_stride is not None else n_out
        y = self._dev(np.full(n_rows * stride, np.float32(-7.25), dtype=np.float32))
        self.H.call(f"matmul_{kind}_rows", dw, dx, y, n_rows, n_out, n_in, stride)
        return y.download(np.float32)

    def rmsnorm(self, x, w, eps):
        dx, dw = self._dev(np.asarray(x, np.float32)), self._dev(np.asarray(w, np.float32))
        y = self.H.DeviceBuffer(x.size * 4)
        self.H.call("rmsnorm", dx, dw, y, x.size, float(eps))
        return y.download(np.float32)

    def rope(self, x, n_heads, pos, head_dim, rotary_dim, theta, style, factors=None):
        dx = self._dev(np.asarray(x, np.float32))
        df = None if factors is None else self._dev(np.asarray(factors, np.float32))
        self.H.call("rope", dx, n_heads, pos, head_dim, rotary_dim, float(theta), C.c_int(style), df)
        return dx.download(np.float32)

    def softmax(self, x):
        dx = self._dev(np.asarray(x, np.float32))
        self.H.call("softmax", dx, x.size)
        return dx.download(np.float32)

    def silu_mul(self, g, u):
        dg, du = self._dev(np.asarray(g, np.float32)), self._dev(np.asarray(u, np.float32))
        out = self.H.DeviceBuffer(g.size * 4)
        self.H.call("silu_mul", dg, du, out, g.size)
        return out.download(np.float32)

    def embedding_row(self, type_id, table, n, index):
        dt = self._dev(np.ascontiguousarray(table))
        out = self.H.DeviceBuffer(n * 4)
        self.H.call("embedding_row", C.c_int(type_id), dt, n, C.c_int64(index), out)
        return out.download(np.float32)

    def attention_kv_heads(self, q, k, v, n_q, n_past, n_head, n_head_kv, head_dim, scale, hb, he, f16=False):
        dq, dk, dv = self._dev(q), self._dev(k), self._dev(v)
        out = self._dev(np.zeros((n_q, n_head, head_dim), dtype=np.float32))
        scores = self.H.DeviceBuffer(max(1, n_q * (n_past + n_q)) * 4)  # the reference's contract, kernels.h:67-75
        self.H.call("attention_kv_heads_f16" if f16 else "attention_kv_heads", dq, dk, dv, out, scores, n_q, n_past,
                    n_head, n_head_kv, head_dim, float(scale), hb, he)
        return out.download(np.float32).reshape(n_q, n_head, head_dim)

    def block_sums(self, type_id, w_row, xq, n_blocks):
        dw, dx = self._dev(w_row), self._dev(xq)
        si = self.H.DeviceBuffer(n_blocks * 4)
        sx = self.H.DeviceBuffer(n_blocks * 4)
        self.H.call("block_sums", C.c_int(type_id), dw, dx, n_blocks, si, sx)
        return si.download(np.int32), sx.download(np.int32)
