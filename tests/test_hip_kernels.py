"""The hip table against the CPU oracle, entry by entry, through the C ABI of libaxon_hip.so.

Integer paths (Q8_0 activation quantization, per-block int32 sums, every matmul with Q8_0
activations) and the float chains the kernels keep in the scalar table's order (float matmuls,
RMSNorm, embedding rows) must be bit-identical, and so must softmax, SiLU and attention, whose
exponential is the host C library's expf restated on the device. Only cos and sin in the
table-less RoPE are held to a few ulp. Patterned on the reference's cross-table tests (tests/unit/test_kernels_neon.cpp,
test_kernels_attention_neon.cpp) and its fixture tests (test_dtype_quant.cpp,
test_kernels_quant.cpp, test_kernels_norm_act.cpp, test_kernels_rope.cpp,
test_kernels_attention.cpp, test_kernels_embedding.cpp)."""
import ctypes as C

import numpy as np
import pytest

from helpers import (BLOCK, GOLDEN, Q4_0, Q4_1, Q6_K, Q8_0, call, golden, golden_blocks)
from tables import CTable, HipTable, QUANT_TYPES, dequantize, random_floats, random_weights, relative_error

pytestmark = pytest.mark.gpu

TYPE_ID = {"q8_0": 8, "q4_0": 2, "q4_1": 3, "q6_k": 14}


@pytest.fixture(scope="module")
def o():
    return CTable("oracle")


@pytest.fixture(scope="module")
def h():
    return HipTable()


def ulp_diff(a, b):
    a = np.ascontiguousarray(a, np.float32).view(np.int32).astype(np.int64)
    b = np.ascontiguousarray(b, np.float32).view(np.int32).astype(np.int64)
    a = np.where(a < 0, -(a & 0x7fffffff), a)
    b = np.where(b < 0, -(b & 0x7fffffff), b)
    return int(np.max(np.abs(a - b))) if a.size else 0


# ---- Q8_0 activation quantization ------------------------------------------------------------

@pytest.mark.parametrize("base", ["row", "act"])
def test_quantize_matches_fixture_bytes(h, base):
    x = golden(f"quant/{base}.f32.axt").ravel()
    want = (GOLDEN / f"quant/{base}.q8_0.bin").read_bytes()
    assert h.quantize_row_q8_0(x).tobytes() == want


def test_quantize_random_and_edge_rows_bit_exact(h, o):
    rng = np.random.default_rng(1)
    rows = [rng.normal(0, 1, 4096).astype(np.float32),
            rng.normal(0, 40, 4096).astype(np.float32),
            np.zeros(64, np.float32),
            np.full(64, 1e-30, np.float32),                       # fp16 underflow of d
            (np.arange(128, dtype=np.float32) - 64) * 0.5,        # exact .5 ties
            np.full(32, 65504.0 * 127, np.float32),               # d overflows fp16
            rng.normal(0, 1e-6, 2048).astype(np.float32)]
    for x in rows:
        assert h.quantize_row_q8_0(x).tobytes() == o.quantize_row_q8_0(x).tobytes()


# ---- per-block integer sums (test hook) ------------------------------------------------------

@pytest.mark.parametrize("kind", QUANT_TYPES)
def test_block_sums_bit_exact(h, o, kind):
    nb = 64
    w = random_weights(kind, 1, nb * 32, 5)
    xq = o.quantize_row_q8_0(random_floats(nb * 32, 6, 3.0))
    si, sx = h.block_sums(TYPE_ID[kind], w, xq, nb)
    want_i = np.zeros(nb, np.int32)
    want_x = np.zeros(nb, np.int32)
    o._c("block_sums", C.c_int(TYPE_ID[kind]), w, xq, nb, want_i, want_x)
    assert np.array_equal(si, want_i)
    if kind == "q4_1":
        assert np.array_equal(sx, want_x)


# ---- matmuls with Q8_0 activations: bit-exact at every row count ---------------------------

@pytest.mark.parametrize("n_in", [32, 96, 576, 2048])
@pytest.mark.parametrize("n_out", [1, 7, 48, 300])
def test_q8_matvec_bit_exact(h, o, n_in, n_out):
    x = random_floats(n_in, n_in + n_out, 4.0)
    xq = o.quantize_row_q8_0(x)
    for kind in QUANT_TYPES:
        w = random_weights(kind, n_out, n_in, n_in * 7 + n_out)
        assert np.array_equal(h.matmul(f"{kind}_q8", w, xq, n_out, n_in),
                              o.matmul(f"{kind}_q8", w, xq, n_out, n_in)), kind


@pytest.mark.parametrize("n_rows", [1, 2, 3, 4, 5, 9, 15, 16, 17, 33, 64, 65])
def test_q8_rows_bit_exact_dot4_and_mfma(h, o, n_rows):
    n_in, n_out = 256, 80
    xs = random_floats(n_rows * n_in, n_rows, 3.0)
    xq = np.concatenate([o.quantize_row_q8_0(xs[i * n_in:(i + 1) * n_in]) for i in range(n_rows)])
    for kind in QUANT_TYPES:
        w = random_weights(kind, n_out, n_in, 40 + n_rows)
        got = h.matmul(f"{kind}_q8", w, xq, n_out, n_in, n_rows=n_rows, y_stride=n_out + 3)
        want = o.matmul(f"{kind}_q8", w, xq, n_out, n_in, n_rows=n_rows, y_stride=n_out + 3)
        assert np.array_equal(got, want), (kind, n_rows)   # sentinels between rows untouched too


@pytest.mark.parametrize("n_rows", [2, 3, 4])
def test_q8_rows_wide_matrix_few_rows_bit_exact(h, o, n_rows):
    """Three and four rows of a matrix wide enough for the decode tile (16384 outputs: 256
    workgroups of 64) take the MFMA tile kernel instead of the dot4 matvec (two rows stay
    there); strided outputs, against the oracle."""
    n_in, n_out = 256, 16384
    xs = random_floats(n_rows * n_in, 60 + n_rows, 3.0)
    xq = np.concatenate([o.quantize_row_q8_0(xs[i * n_in:(i + 1) * n_in]) for i in range(n_rows)])
    for kind in QUANT_TYPES:
        w = random_weights(kind, n_out, n_in, 50 + n_rows)
        got = h.matmul(f"{kind}_q8", w, xq, n_out, n_in, n_rows=n_rows, y_stride=n_out + 5)
        want = o.matmul(f"{kind}_q8", w, xq, n_out, n_in, n_rows=n_rows, y_stride=n_out + 5)
        assert np.array_equal(got, want), (kind, n_rows)


@pytest.mark.parametrize("kind", QUANT_TYPES)
def test_q8_rows_long_k_and_unaligned_weights(h, o, kind):
    # K = 8192 spans several LDS chunks of the MFMA path, which also takes 3 and 4 rows at this
    # length (1 and 2 stay on the dot4 kernel). The weight pointer is then moved 2 bytes off any
    # 4-byte boundary, as a column chunk of an odd block count leaves it (matmul_columns passes
    # base + begin * row_bytes, llama.cpp:36-37), which sends every row count to the dot4 kernel.
    import axon_hip as H
    n_in, n_out, n_rows = 8192, 40, 20
    xs = random_floats(n_rows * n_in, 77, 2.0)
    xq = np.concatenate([o.quantize_row_q8_0(xs[i * n_in:(i + 1) * n_in]) for i in range(n_rows)])
    w = random_weights(kind, n_out, n_in, 78)
    for rows in (1, 2, 3, 4, n_rows):
        want = o.matmul(f"{kind}_q8", w, xq[: rows * n_in // 32], n_out, n_in, n_rows=rows)
        assert np.array_equal(h.matmul(f"{kind}_q8", w, xq[: rows * n_in // 32], n_out, n_in, n_rows=rows), want)
        raw = w.tobytes()
        buf = H.DeviceBuffer(len(raw) + 16)
        buf.upload(np.frombuffer(raw, np.uint8), offset=2)
        dx = H.DeviceBuffer.of(xq[: rows * n_in // 32])
        y = H.DeviceBuffer.of(np.zeros(rows * n_out, np.float32))
        H.call(f"matmul_{kind}_q8_rows", buf.at(2), dx, y, rows, n_out, n_in, n_out)
        assert np.array_equal(y.download(np.float32), want), (kind, rows)


@pytest.mark.parametrize("n_rows", [5, 8, 16, 24, 32, 40, 64])
@pytest.mark.parametrize("n_in", [896, 2048])
def test_q8_fused_segments_few_rows_bit_exact(o, n_rows, n_in):
    """The few-rows MFMA path (5..64 activation rows): three segments of uneven widths in one
    grid, a last K chunk of 12 blocks at n_in 896, y_stride past n_out with the sentinels between
    rows untouched, and accumulate (y += W x) — each output equal to the oracle's row by row."""
    import axon_hip as H
    n_out = [300, 7, 64]
    stride = [n + 5 for n in n_out]
    xs = random_floats(n_rows * n_in, n_rows + n_in, 3.0)
    xq = np.concatenate([o.quantize_row_q8_0(xs[i * n_in:(i + 1) * n_in]) for i in range(n_rows)])
    dx = H.DeviceBuffer.of(xq)
    for kind in QUANT_TYPES:
        ws = [random_weights(kind, n, n_in, 100 * j + n_rows) for j, n in enumerate(n_out)]
        for accumulate in (0, 1):
            base = [random_floats(n_rows * st, 7 + j, 1.0) for j, st in enumerate(stride)]
            dws = [H.DeviceBuffer.of(w) for w in ws]
            dys = [H.DeviceBuffer.of(b) for b in base]
            n = len(ws)
            H.check(H.lib().axon_hip_matmul_q8_fused(
                C.c_int(TYPE_ID[kind]), C.c_void_p(dx.ptr), C.c_size_t(n_rows), C.c_size_t(n_in), C.c_size_t(n),
                (C.c_void_p * n)(*[b.ptr for b in dws]), (C.c_void_p * n)(*[b.ptr for b in dys]),
                (C.c_size_t * n)(*n_out), (C.c_size_t * n)(*stride), C.c_int(accumulate)), "matmul_q8_fused")
            for j in range(n):
                got = dys[j].download(np.float32).reshape(n_rows, stride[j])
                want = o.matmul(f"{kind}_q8", ws[j], xq, n_out[j], n_in, n_rows=n_rows,
                                y_stride=n_out[j]).reshape(n_rows, n_out[j])
                if accumulate:
                    want = base[j].reshape(n_rows, stride[j])[:, :n_out[j]] + want
                assert np.array_equal(got[:, :n_out[j]], want), (kind, j, accumulate)
                assert np.array_equal(got[:, n_out[j]:], base[j].reshape(n_rows, stride[j])[:, n_out[j]:])


@pytest.mark.parametrize("n_rows", [5, 16, 17, 32])
def test_q8_fused_segments_wide_decode_bit_exact(o, n_rows):
    """Decode batches (5..32 rows) on a matrix wide enough for the tile kernel with 16 or 32
    activation rows per workgroup (64 weight rows per workgroup up to 16 rows, 32 above):
    segments of 16384, 7 and 300 rows (partial weight tiles), a last K chunk of 12 blocks, the
    sentinels past n_out untouched, and accumulate — each output equal to the oracle's."""
    import axon_hip as H
    n_in, n_out = 896, [16384, 7, 300]
    stride = [n + 3 for n in n_out]
    xs = random_floats(n_rows * n_in, 5 * n_rows + n_in, 3.0)
    xq = np.concatenate([o.quantize_row_q8_0(xs[i * n_in:(i + 1) * n_in]) for i in range(n_rows)])
    dx = H.DeviceBuffer.of(xq)
    for kind in QUANT_TYPES:
        ws = [random_weights(kind, n, n_in, 300 * j + n_rows) for j, n in enumerate(n_out)]
        wants = [o.matmul(f"{kind}_q8", ws[j], xq, n_out[j], n_in, n_rows=n_rows,
                          y_stride=n_out[j]).reshape(n_rows, n_out[j]) for j in range(len(ws))]
        dws = [H.DeviceBuffer.of(w) for w in ws]
        for accumulate in (0, 1):
            base = [random_floats(n_rows * st, 9 + j, 1.0) for j, st in enumerate(stride)]
            dys = [H.DeviceBuffer.of(b) for b in base]
            n = len(ws)
            H.check(H.lib().axon_hip_matmul_q8_fused(
                C.c_int(TYPE_ID[kind]), C.c_void_p(dx.ptr), C.c_size_t(n_rows), C.c_size_t(n_in), C.c_size_t(n),
                (C.c_void_p * n)(*[b.ptr for b in dws]), (C.c_void_p * n)(*[b.ptr for b in dys]),
                (C.c_size_t * n)(*n_out), (C.c_size_t * n)(*stride), C.c_int(accumulate)), "matmul_q8_fused")
            for j in range(n):
                got = dys[j].download(np.float32).reshape(n_rows, stride[j])
                want = wants[j]
                if accumulate:
                    want = base[j].reshape(n_rows, stride[j])[:, :n_out[j]] + want
                assert np.array_equal(got[:, :n_out[j]], want), (kind, j, accumulate)
                assert np.array_equal(got[:, n_out[j]:], base[j].reshape(n_rows, stride[j])[:, n_out[j]:])


@pytest.mark.parametrize("n_rows, n_in, n_out", [(65, 896, [300, 7, 64]), (77, 2048, [300, 7, 64]),
                                                  (200, 896, [1152, 896, 40]), (576, 896, [4096, 1024, 1024]),
                                                  (130, 4864, [896, 33, 64]), (40, 896, [32768, 7, 64]),
                                                  (64, 256, [32800])])
def test_q8_fused_segments_many_rows_bit_exact(o, n_rows, n_in, n_out):
    """The tile MFMA path (65 rows and more, prefill and mixed passes; 33 to 64 rows on matrices
    of 512 or more 64-row tiles, the last two shapes): segments in one grid with 32- and 64-row
    weight tiles,
    partial activation and weight tiles, a last K chunk shorter than 16 blocks, y_stride past
    n_out with the sentinels between rows untouched, and accumulate (y += W x) — each output
    equal to the oracle's row by row."""
    import axon_hip as H
    stride = [n + 3 for n in n_out]
    xs = random_floats(n_rows * n_in, n_rows + n_in, 3.0)
    xq = np.concatenate([o.quantize_row_q8_0(xs[i * n_in:(i + 1) * n_in]) for i in range(n_rows)])
    dx = H.DeviceBuffer.of(xq)
    for kind in QUANT_TYPES:
        ws = [random_weights(kind, n, n_in, 100 * j + n_rows) for j, n in enumerate(n_out)]
        wants = [o.matmul(f"{kind}_q8", ws[j], xq, n_out[j], n_in, n_rows=n_rows,
                          y_stride=n_out[j]).reshape(n_rows, n_out[j]) for j in range(len(ws))]
        for accumulate in (0, 1):
            base = [random_floats(n_rows * st, 7 + j, 1.0) for j, st in enumerate(stride)]
            dws = [H.DeviceBuffer.of(w) for w in ws]
            dys = [H.DeviceBuffer.of(b) for b in base]
            n = len(ws)
            H.check(H.lib().axon_hip_matmul_q8_fused(
                C.c_int(TYPE_ID[kind]), C.c_void_p(dx.ptr), C.c_size_t(n_rows), C.c_size_t(n_in), C.c_size_t(n),
                (C.c_void_p * n)(*[b.ptr for b in dws]), (C.c_void_p * n)(*[b.ptr for b in dys]),
                (C.c_size_t * n)(*n_out), (C.c_size_t * n)(*stride), C.c_int(accumulate)), "matmul_q8_fused")
            for j in range(n):
                got = dys[j].download(np.float32).reshape(n_rows, stride[j])
                want = wants[j]
                if accumulate:
                    want = base[j].reshape(n_rows, stride[j])[:, :n_out[j]] + want
                assert np.array_equal(got[:, :n_out[j]], want), (kind, j, accumulate)
                assert np.array_equal(got[:, n_out[j]:], base[j].reshape(n_rows, stride[j])[:, n_out[j]:])


@pytest.mark.parametrize("n_rows, n_in, n_ff", [(65, 896, 4864), (130, 2048, 1024), (512, 256, 96),
                                                 (1, 256, 8192), (5, 512, 8192), (16, 256, 8224), (17, 256, 8192),
                                                 (32, 512, 8192), (48, 256, 8192), (64, 256, 8192), (16, 896, 4864),
                                                 (40, 896, 4864), (7, 256, 4096)])
def test_q8_swiglu_tile_bit_exact(o, n_rows, n_in, n_ff):
    """gate|up with the SwiGLU product and down's Q8_0 input in the tile kernel's epilogue
    (axon_hip_matmul_q8_swiglu): the float product and the Q8_0 blocks equal, bit for bit,
    the unfused device path (matmul_q8_fused of both weights, then silu_mul_rows), whose parts
    are pinned to the oracle elsewhere; and the product and its blocks equal the oracle's
    matmuls, silu_mul and quantize_row_q8_0. Decode-sized calls (up to 64 rows: tiles of 16, 32
    and 64 activation rows, the first two meeting gate and up in LDS) run when the FFN gives
    at least 128 workgroups (n_ff 4096 and up)."""
    import axon_hip as H
    xs = random_floats(n_rows * n_in, n_rows + n_ff, 3.0)
    xq = np.concatenate([o.quantize_row_q8_0(xs[i * n_in:(i + 1) * n_in]) for i in range(n_rows)])
    dx = H.DeviceBuffer.of(xq)
    for kind in QUANT_TYPES:
        wg = random_weights(kind, n_ff, n_in, 11 + n_rows)
        wu = random_weights(kind, n_ff, n_in, 12 + n_rows)
        g = o.matmul(f"{kind}_q8", wg, xq, n_ff, n_in, n_rows=n_rows, y_stride=n_ff).reshape(n_rows, n_ff)
        u = o.matmul(f"{kind}_q8", wu, xq, n_ff, n_in, n_rows=n_rows, y_stride=n_ff).reshape(n_rows, n_ff)
        prod = np.stack([o.silu_mul(g[r], u[r]) for r in range(n_rows)])
        want_q = np.concatenate([o.quantize_row_q8_0(prod[r]) for r in range(n_rows)])
        dwg, dwu = H.DeviceBuffer.of(wg), H.DeviceBuffer.of(wu)
        out = H.DeviceBuffer.of(np.full(n_rows * n_ff, np.float32(-3.5), np.float32))
        outq = H.DeviceBuffer(want_q.nbytes)
        H.check(H.lib().axon_hip_matmul_q8_swiglu(
            C.c_int(TYPE_ID[kind]), C.c_void_p(dx.ptr), C.c_size_t(n_rows), C.c_size_t(n_in), C.c_void_p(dwg.ptr),
            C.c_void_p(dwu.ptr), C.c_size_t(n_ff), C.c_void_p(out.ptr), C.c_void_p(outq.ptr)), "matmul_q8_swiglu")
        got = out.download(np.float32).reshape(n_rows, n_ff)
        got_q = outq.download(np.uint8, want_q.nbytes)
        # The unfused device path.
        dg, du = H.DeviceBuffer(4 * n_rows * n_ff), H.DeviceBuffer(4 * n_rows * n_ff)
        H.check(H.lib().axon_hip_matmul_q8_fused(
            C.c_int(TYPE_ID[kind]), C.c_void_p(dx.ptr), C.c_size_t(n_rows), C.c_size_t(n_in), C.c_size_t(2),
            (C.c_void_p * 2)(dwg.ptr, dwu.ptr), (C.c_void_p * 2)(dg.ptr, du.ptr), (C.c_size_t * 2)(n_ff, n_ff),
            (C.c_size_t * 2)(n_ff, n_ff), C.c_int(0)), "matmul_q8_fused")
        ref_out, ref_q = H.DeviceBuffer(4 * n_rows * n_ff), H.DeviceBuffer(want_q.nbytes)
        H.call("silu_mul_rows", dg, du, ref_out, ref_q, n_ff, n_rows)
        assert np.array_equal(got.view(np.uint32), ref_out.download(np.uint32, n_rows * n_ff).reshape(n_rows, n_ff)), kind
        assert got_q.tobytes() == ref_q.download(np.uint8, want_q.nbytes).tobytes(), kind
        assert np.array_equal(got, prod), kind
        assert got_q.tobytes() == want_q.tobytes(), kind
    # A decode-sized call whose FFN gives 127 workgroups: refused, nothing launched.
    with pytest.raises(H.HipError, match="swiglu"):
        H.check(H.lib().axon_hip_matmul_q8_swiglu(C.c_int(2), C.c_void_p(dx.ptr), C.c_size_t(64), C.c_size_t(n_in),
                                                  C.c_void_p(dx.ptr), C.c_void_p(dx.ptr), C.c_size_t(4064), None,
                                                  C.c_void_p(dx.ptr)), "matmul_q8_swiglu")


@pytest.mark.parametrize("name,dt", [("q8_0", Q8_0), ("q4_0", Q4_0), ("q4_1", Q4_1)])
def test_q8_matmul_fixtures(h, name, dt):
    # The reference's float64 integer-dot fixtures (test_kernels_quant.cpp:50-84, 101-134).
    w = golden_blocks(f"quant/matmul_{name}.w.bin", dt)
    xq = golden_blocks(f"quant/matmul_{name}.xq.bin", Q8_0)
    want = golden(f"quant/matmul_{name}.yq.axt").ravel()
    n_out, n_in = want.size, xq.size * 32
    got = h.matmul(f"{name}_q8", w, xq, n_out, n_in)
    assert np.max(np.abs(got - want) / (np.abs(want) + 1e-6)) < 1e-5


# ---- float matmuls: bit-exact -----------------------------------------------------------------

@pytest.mark.parametrize("n_in,n_out", [(64, 5), (320, 33)])
def test_float_matmuls_bit_exact(h, o, n_in, n_out):
    wf = random_floats(n_out * n_in, 3)
    w16 = wf.astype(np.float16).view(np.uint16)
    wb = (wf.view(np.uint32) >> 16).astype(np.uint16)
    x = random_floats(n_in, 4)
    xs = random_floats(3 * n_in, 5)
    for kind, w in (("f32", wf), ("f16", w16), ("bf16", wb)):
        assert np.array_equal(h.matmul(kind, w, x, n_out, n_in), o.matmul(kind, w, x, n_out, n_in)), kind
        assert np.array_equal(h.matmul(kind, w, xs, n_out, n_in, n_rows=3, y_stride=n_out + 2),
                              o.matmul(kind, w, xs, n_out, n_in, n_rows=3, y_stride=n_out + 2)), kind
    for kind in QUANT_TYPES:
        w = random_weights(kind, n_out, n_in, 6)
        assert np.array_equal(h.matmul(kind, w, x, n_out, n_in), o.matmul(kind, w, x, n_out, n_in)), kind
        assert np.array_equal(h.matmul(kind, w, xs, n_out, n_in, n_rows=3),
                              o.matmul(kind, w, xs, n_out, n_in, n_rows=3)), kind


@pytest.mark.parametrize("name", ["matmul_f32", "matmul_f16", "matmul_bf16", "matmul_f32_odd"])
def test_float_matmul_fixtures(h, name):
    kind = name.split("_")[1]
    w = golden(f"kernels/{name}.w.axt")
    x = golden(f"kernels/{name}.x.axt").ravel()
    want = golden(f"kernels/{name}.y.axt").ravel()
    got = h.matmul(kind, w, x, want.size, x.size)
    assert np.max(np.abs(got - want)) <= 1e-5 * max(1.0, np.max(np.abs(want)))


# ---- Q6_K: float path, bit-exact (the dequantized value is exact in float) -----------------

@pytest.mark.parametrize("n_in,n_out,n_rows", [(256, 9, 1), (2048, 300, 1), (2048, 64, 3), (2048, 40, 9),
                                               (768, 70, 2), (8192, 65, 1)])
def test_q6_k_bit_exact(h, o, n_in, n_out, n_rows):
    w = random_weights("q6_k", n_out, n_in, n_in + n_out)
    x = random_floats(n_rows * n_in, 9)
    if n_rows == 1:
        assert np.array_equal(h.matmul("q6_k", w, x, n_out, n_in), o.matmul("q6_k", w, x, n_out, n_in))
    else:
        got = h.matmul("q6_k", w, x, n_out, n_in, n_rows=n_rows, y_stride=n_out + 1)
        want = o.matmul("q6_k", w, x, n_out, n_in, n_rows=n_rows, y_stride=n_out + 1)
        assert np.array_equal(got, want)


def test_q6_k_unaligned_weights(h, o):
    # A weight pointer 2 bytes off a 4-byte boundary flips which super-blocks start aligned.
    import axon_hip as H
    n_in, n_out = 1280, 33
    w = random_weights("q6_k", n_out, n_in, 5)
    x = random_floats(n_in, 6)
    raw = np.frombuffer(w.tobytes(), np.uint8)
    buf = H.DeviceBuffer(raw.size + 16)
    buf.upload(raw, offset=2)
    dx = H.DeviceBuffer.of(x)
    y = H.DeviceBuffer(n_out * 4)
    H.call("matmul_q6_k", buf.at(2), dx, y, n_out, n_in)
    assert np.array_equal(y.download(np.float32), o.matmul("q6_k", w, x, n_out, n_in))


def test_q6_k_fixture(h):
    w = golden_blocks("quant/matmul_q6_k.w.bin", Q6_K)
    x = golden("quant/matmul_q6_k.x.axt").ravel()
    want = golden("quant/matmul_q6_k.y.axt").ravel()
    got = h.matmul("q6_k", w, x, want.size, x.size)
    assert np.max(np.abs(got - want)) <= 1e-3 * max(1.0, np.max(np.abs(want)))


# ---- norms, activations, rope, softmax -------------------------------------------------------

@pytest.mark.parametrize("n", [1, 64, 576, 2048, 5000])
def test_rmsnorm_bit_exact(h, o, n):
    x = random_floats(n, n, 3.0)
    w = 1.0 + random_floats(n, n + 1, 0.1)
    assert np.array_equal(h.rmsnorm(x, w, 1e-5), o.rmsnorm(x, w, 1e-5))


@pytest.mark.parametrize("n", [1, 64])
def test_rmsnorm_fixtures(h, n):
    x, w, y = (golden(f"kernels/rmsnorm_{n}.{s}.axt").ravel() for s in "xwy")
    assert np.max(np.abs(h.rmsnorm(x, w, 1e-5) - y)) < 1e-5


def test_silu_mul_bit_exact(h, o):
    """SiLU through the host C library's expf (glibc 2.35, restated on the device): bit-exact
    against the oracle, which calls expf. The gates include a dense sweep of every 97th float in
    [-2^-9, 2^-9], where that expf is not correctly rounded (about 1 argument in 10^4 there
    differs from the once-rounded binary64 exp)."""
    g = random_floats(5000, 1, 12.0)
    u = random_floats(5000, 2, 3.0)
    assert np.array_equal(h.silu_mul(g, u), o.silu_mul(g, u))
    lo, hi = np.float32(2.0 ** -9).view(np.uint32), np.float32(2.0 ** -20).view(np.uint32)
    mags = np.arange(hi, lo, 97, dtype=np.uint32).view(np.float32)
    gs = np.concatenate([mags, -mags]).astype(np.float32)
    ones = np.ones_like(gs)
    assert np.array_equal(h.silu_mul(gs, ones), o.silu_mul(gs, ones))
    gg, uu, want = (golden(f"kernels/silu_mul.{s}.axt").ravel() for s in ("gate", "up", "out"))
    assert np.max(np.abs(h.silu_mul(gg, uu) - want)) < 1e-5


@pytest.mark.parametrize("n", [1, 5, 64, 3000])
def test_softmax_bit_exact(h, o, n):
    x = random_floats(n, n, 20.0)
    assert np.array_equal(h.softmax(x), o.softmax(x))
    # Near-ties of the maximum: arguments of expf within 2^-9 of zero.
    rng = np.random.default_rng(n + 1)
    y = (np.float32(3.0) - np.abs(rng.standard_normal(n)).astype(np.float32) * np.float32(1e-3)).astype(np.float32)
    assert np.array_equal(h.softmax(y), o.softmax(y))
    if n in (1, 5, 64):
        xx, yy = golden(f"kernels/softmax_{n}.x.axt").ravel(), golden(f"kernels/softmax_{n}.y.axt").ravel()
        assert np.max(np.abs(h.softmax(xx) - yy)) < 1e-5


@pytest.mark.parametrize("name,style,theta,factors", [("rope_normal", 0, 10000.0, False),
                                                      ("rope_neox", 1, 1000000.0, False),
                                                      ("rope_llama3", 0, 500000.0, True)])
def test_rope_fixtures_and_oracle(h, o, name, style, theta, factors):
    x = golden(f"kernels/{name}.x.axt")
    pos = golden(f"kernels/{name}.pos.axt").ravel()
    y = golden(f"kernels/{name}.y.axt")
    f = golden(f"kernels/{name}.factors.axt").ravel() if factors else None
    n_rows, n_heads, hd = x.shape
    for r in range(n_rows):
        got = h.rope(x[r], n_heads, int(pos[r]), hd, hd, theta, style, f).reshape(n_heads, hd)
        assert np.max(np.abs(got - y[r])) < 1e-4 * max(1.0, float(pos[r]) / 100)
        want = o.rope(x[r], n_heads, int(pos[r]), hd, hd, theta, style, f)
        # cos/sin evaluated on the device in double: the float results agree to an ulp or two
        assert np.max(np.abs(got - want)) <= 4 * np.finfo(np.float32).eps * max(1.0, np.max(np.abs(want)))


# ---- embedding rows: exact for every type -----------------------------------------------------

@pytest.mark.parametrize("name,type_id,dt", [("q8_0", 8, Q8_0), ("q4_0", 2, Q4_0), ("q4_1", 3, Q4_1),
                                             ("q6_k", 14, Q6_K)])
def test_quantized_embedding_exact(h, o, name, type_id, dt):
    table = golden_blocks(f"quant/embedding_{name}.table.bin", dt)
    idx = golden(f"quant/embedding_{name}.index.axt").ravel()
    rows = golden(f"quant/embedding_{name}.rows.axt")
    n = rows.shape[-1]
    for i, r in enumerate(idx):
        got = h.embedding_row(type_id, table, n, int(r))
        assert np.array_equal(got, rows[i])
        assert np.array_equal(got, o.embedding_row(type_id, table, n, int(r)))


@pytest.mark.parametrize("name,type_id", [("f32", 0), ("f16", 1), ("bf16", 30)])
def test_float_embedding_exact(h, name, type_id):
    table = golden(f"kernels/embedding_{name}.table.axt")
    idx = golden(f"kernels/embedding_{name}.index.axt").ravel()
    rows = golden(f"kernels/embedding_{name}.rows.axt")
    n = rows.shape[-1]
    for i, r in enumerate(idx):
        assert np.array_equal(h.embedding_row(type_id, table, n, int(r)), rows[i])


# ---- attention -----------------------------------------------------------------------------------

@pytest.mark.parametrize("n_q,n_past,n_head,n_kv,hd", [(1, 0, 4, 2, 64), (1, 37, 9, 3, 64), (5, 11, 8, 2, 64),
                                                       (16, 100, 32, 8, 64), (3, 600, 14, 2, 64),
                                                       (2, 5, 4, 4, 16), (1, 3000, 4, 1, 64),
                                                       (37, 20, 9, 3, 64), (33, 5, 14, 2, 64), (18, 300, 32, 4, 64),
                                                       (130, 0, 32, 8, 64), (300, 0, 32, 8, 64), (260, 40, 32, 4, 64)])
def test_attention_matches_oracle(h, o, n_q, n_past, n_head, n_kv, hd):
    rng = np.random.default_rng(n_q * 1000 + n_past)
    total = n_past + n_q
    q = rng.normal(0, 1, (n_q, n_head, hd)).astype(np.float32)
    k = rng.normal(0, 1, (total, n_kv, hd)).astype(np.float32)
    v = rng.normal(0, 1, (total, n_kv, hd)).astype(np.float32)
    scale = 1.0 / np.sqrt(hd)
    got = h.attention_kv_heads(q, k, v, n_q, n_past, n_head, n_kv, hd, scale, 0, n_head)
    want = o.attention_kv_heads(q, k, v, n_q, n_past, n_head, n_kv, hd, scale, 0, n_head)
    # The exponential is the host's expf; the double sum of the softmax is reduced as a fixed
    # tree, which can differ from the sequential sum only when 1 / sum sits within a double ulp
    # of a float rounding midpoint.
    assert np.array_equal(got, want)
    # head ranges compose (test_kernels_attention.cpp:187-210)
    part = h.attention_kv_heads(q, k, v, n_q, n_past, n_head, n_kv, hd, scale, 1, n_head)
    assert np.array_equal(part[:, 1:], got[:, 1:])
    # the fp16 cache variant widens exactly
    k16, v16 = k.astype(np.float16).view(np.uint16), v.astype(np.float16).view(np.uint16)
    got16 = h.attention_kv_heads(q, k16, v16, n_q, n_past, n_head, n_kv, hd, scale, 0, n_head, f16=True)
    want16 = o.attention_kv_heads(q, k16, v16, n_q, n_past, n_head, n_kv, hd, scale, 0, n_head, f16=True)
    assert np.array_equal(got16, want16)


@pytest.mark.parametrize("name,seq,nh,nkv,hd", [("attention_s8_h4_kv2_d16", 8, 4, 2, 16),
                                                ("attention_s1_h2_kv1_d8", 1, 2, 1, 8),
                                                ("attention_s5_h2_kv1_d8", 5, 2, 1, 8)])
def test_attention_fixtures(h, name, seq, nh, nkv, hd):
    q, k, v, want = (golden(f"kernels/{name}.{s}.axt") for s in ("q", "k", "v", "out"))
    got = h.attention_kv_heads(q, k, v, seq, 0, nh, nkv, hd, 1.0 / np.sqrt(hd), 0, nh)
    assert np.max(np.abs(got - want.reshape(got.shape))) < 1e-5


def test_attention_over_one_position_returns_its_value(h):
    # attention.cpp closed form (test_kernels_attention.cpp:55-76)
    rng = np.random.default_rng(3)
    q = rng.normal(0, 1, (1, 4, 64)).astype(np.float32)
    k = rng.normal(0, 1, (1, 2, 64)).astype(np.float32)
    v = rng.normal(0, 1, (1, 2, 64)).astype(np.float32)
    got = h.attention_kv_heads(q, k, v, 1, 0, 4, 2, 64, 0.125, 0, 4)
    assert np.array_equal(got[0, 0], v[0, 0]) and np.array_equal(got[0, 3], v[0, 1])


@pytest.mark.parametrize("f16", [False, True])
def test_attention_heads_stay_within_the_reference_scratch(o, f16):
    """The reference's scratch contract (kernels.h:67-75): a call over heads [h, h + 1), or over
    every head, with scores of n_q * (n_past + n_q) floats only, at a context whose scores spill
    out of LDS (3000 positions, a GQA group of 8, as LlamaModel calls it per head,
    llama.cpp:540-556). The floats after the scratch are a guard that must stay untouched, heads
    outside the range keep their sentinel outputs, and every head equals the oracle."""
    import axon_hip as H
    n_q, n_past, n_head, n_kv, hd = 2, 3000, 32, 4, 64
    total = n_past + n_q
    rng = np.random.default_rng(31 + int(f16))
    q = rng.normal(0, 1, (n_q, n_head, hd)).astype(np.float32)
    k = rng.normal(0, 1, (total, n_kv, hd)).astype(np.float32)
    v = rng.normal(0, 1, (total, n_kv, hd)).astype(np.float32)
    if f16:
        k, v = k.astype(np.float16).view(np.uint16), v.astype(np.float16).view(np.uint16)
    want = o.attention_kv_heads(q, k, v, n_q, n_past, n_head, n_kv, hd, 0.125, 0, n_head, f16=f16)
    guard = np.full(4096, np.float32(-7.25), np.float32)
    dq, dk, dv = H.DeviceBuffer.of(q), H.DeviceBuffer.of(k), H.DeviceBuffer.of(v)
    scores = H.DeviceBuffer(4 * (n_q * total + guard.size))
    scores.upload(guard, offset=4 * n_q * total)
    entry = "attention_kv_heads_f16" if f16 else "attention_kv_heads"
    for hb, he in ((5, 6), (16, 17), (31, 32), (0, n_head)):
        sentinel = np.full((n_q, n_head, hd), np.float32(9.5), np.float32)
        out = H.DeviceBuffer.of(sentinel)
        H.call(entry, dq, dk, dv, out, scores, n_q, n_past, n_head, n_kv, hd, 0.125, hb, he)
        got = out.download(np.float32).reshape(n_q, n_head, hd)
        assert np.array_equal(got[:, hb:he], want[:, hb:he]), (hb, he)
        assert np.array_equal(np.delete(got, np.s_[hb:he], axis=1), np.delete(sentinel, np.s_[hb:he], axis=1))
        assert np.array_equal(scores.download(np.float32, guard.size, 4 * n_q * total), guard), (hb, he)


@pytest.mark.parametrize("seq,n_past,n_head,n_kv", [(7, 0, 8, 2), (1, 900, 14, 2), (3, 2500, 32, 8), (2, 3000, 16, 2)])
def test_attention_and_attention_kv_entries(o, seq, n_past, n_head, n_kv):
    """The table's attention (a whole sequence, no cache: kernels.h:60-66) and attention_kv (every
    head, kernels.h:67-75) entries against the oracle's, bit for bit, within the reference's
    scratch size."""
    import axon_hip as H
    hd = 64
    total = n_past + seq
    rng = np.random.default_rng(seq + n_past)
    q = rng.normal(0, 1, (seq, n_head, hd)).astype(np.float32)
    k = rng.normal(0, 1, (total, n_kv, hd)).astype(np.float32)
    v = rng.normal(0, 1, (total, n_kv, hd)).astype(np.float32)
    dq, dk, dv = H.DeviceBuffer.of(q), H.DeviceBuffer.of(k), H.DeviceBuffer.of(v)
    scores = H.DeviceBuffer(4 * seq * total)
    out = H.DeviceBuffer(q.nbytes)
    want = np.zeros_like(q)
    osc = np.zeros(seq * total, np.float32)
    if n_past == 0:
        H.call("attention", dq, dk, dv, out, scores, seq, n_head, n_kv, hd, 0.125)
        call(o.lib, "ora_attention", q, k, v, want, osc, seq, n_head, n_kv, hd, 0.125)
    else:
        H.call("attention_kv", dq, dk, dv, out, scores, seq, n_past, n_head, n_kv, hd, 0.125)
        call(o.lib, "ora_attention_kv", q, k, v, want, osc, seq, n_past, n_head, n_kv, hd, 0.125)
    assert np.array_equal(out.download(np.float32).reshape(q.shape), want)


# ---- ragged rows entry (one launch over several sequences' caches) -----------------------------

@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("n_head,n_kv,lens", [(32, 8, [1, 37, 600, 130]), (14, 2, [5, 1025]), (9, 3, [64] * 40),
                                              (32, 4, [2000, 17, 33]), (32, 8, [2304])])
def test_attention_rows_ragged_matches_oracle(o, h, n_head, n_kv, lens, f16):
    """axon_hip_attention_rows over a pool of caches, each row at its own length (decode-shaped
    batches take the two-kernel path; 40 rows x 3 kv heads take the fused one), against the
    oracle's attention_kv_heads (_f16 for a pool of fp16 bit patterns) per sequence."""
    import axon_hip as H
    hd = 64
    rng = np.random.default_rng(sum(lens) + int(f16))
    max_ctx = max(lens) + 3
    n = len(lens)
    row = n_kv * hd
    pool = rng.normal(0, 1, (n, 2, max_ctx, row)).astype(np.float32)     # per sequence: K rows, V rows
    if f16:
        pool[..., ::7] *= np.float32(1e-6)   # fp16 subnormals among the keys and values
        pool = pool.astype(np.float16).view(np.uint16)
    q = rng.normal(0, 1, (n, n_head * hd)).astype(np.float32)
    slot = pool[0].size
    d_pool = H.DeviceBuffer.of(pool)
    d_q = H.DeviceBuffer.of(q)
    d_out = H.DeviceBuffer(q.nbytes)
    off = np.arange(n, dtype=np.int64) * slot
    d_off = H.DeviceBuffer.of(off)
    d_vis = H.DeviceBuffer.of(np.array(lens, np.int32))
    args = H.AttentionRowsArgs(q=d_q.ptr, out=d_out.ptr, q_stride=n_head * hd, out_stride=n_head * hd, kv=d_pool.ptr,
                               k_off=d_off.ptr, v_off=d_off.ptr, n_vis=d_vis.ptr, k_layer_off=0,
                               v_layer_off=max_ctx * row, n_past=0, n_head=n_head, n_kv=n_kv, head_dim=hd,
                               scale=0.125, f16=int(f16), scratch=0, max_vis=max(lens))
    need = H.lib().axon_hip_attention_scratch_floats(C.byref(args), C.c_size_t(n))
    scratch = H.DeviceBuffer(max(need, 1) * 4)
    args.scratch = scratch.ptr if need else 0
    H.check(H.lib().axon_hip_attention_rows(C.byref(args), C.c_size_t(n)), "attention_rows")
    got = d_out.download(np.float32).reshape(n, n_head, hd)
    for i, L in enumerate(lens):
        want = o.attention_kv_heads(q[i].reshape(1, n_head, hd), pool[i, 0, :L].copy(), pool[i, 1, :L].copy(), 1, L - 1,
                                    n_head, n_kv, hd, 0.125, 0, n_head, f16=f16)[0]
        assert np.array_equal(got[i], want), i


@pytest.mark.parametrize("f16", [False, True])
@pytest.mark.parametrize("n_head,n_kv,chunk", [(32, 8, (300, 45)), (32, 8, (40, 300)), (9, 3, (0, 700)),
                                               (14, 2, (600, 520)), (32, 4, (120, 300))])
def test_attention_rows_chunk_among_decode_rows(o, h, n_head, n_kv, chunk, f16):
    """A mixed pass's attention: decode rows of three sequences around the prefill chunk of a
    fourth (rows n_past .. n_past + m - 1 of that sequence, each seeing its own prefix), with the
    Q8_0 output blocks (wo's input) requested. Blocks of rows that share one sequence's K/V read
    it once (blocks of 4, 2 or 1 rows by the row count); blocks that straddle sequences, or whose
    scores outgrow the launch's LDS (the last rows of the 14/2 chunk), run one row at a time.
    Every output row and every Q8_0 block equal the oracle's."""
    import axon_hip as H
    hd = 64
    n_past, m = chunk
    dec = [700, 41, 900]
    lens = [dec[0], n_past + m, dec[1], dec[2]]
    rng = np.random.default_rng(n_head + n_past + m + int(f16))
    max_ctx = max(lens) + 3
    row = n_kv * hd
    pool = rng.normal(0, 1, (4, 2, max_ctx, row)).astype(np.float32)
    if f16:
        pool = pool.astype(np.float16).view(np.uint16)
    # rows: decode seq 0, the chunk of seq 1 (m rows), decode seqs 2 and 3
    seq_of = [0] + [1] * m + [2, 3]
    vis = [lens[0]] + [n_past + i + 1 for i in range(m)] + [lens[2], lens[3]]
    n = len(seq_of)
    q = rng.normal(0, 1, (n, n_head * hd)).astype(np.float32)
    slot = pool[0].size
    d_pool, d_q = H.DeviceBuffer.of(pool), H.DeviceBuffer.of(q)
    d_out = H.DeviceBuffer(q.nbytes)
    nbq = n_head * hd // 32
    d_outq = H.DeviceBuffer(n * nbq * 34)
    d_off = H.DeviceBuffer.of(np.array(seq_of, np.int64) * slot)
    d_vis = H.DeviceBuffer.of(np.array(vis, np.int32))
    args = H.AttentionRowsArgs(q=d_q.ptr, out=d_out.ptr, q_stride=n_head * hd, out_stride=n_head * hd, kv=d_pool.ptr,
                               k_off=d_off.ptr, v_off=d_off.ptr, n_vis=d_vis.ptr, k_layer_off=0,
                               v_layer_off=max_ctx * row, n_past=0, n_head=n_head, n_kv=n_kv, head_dim=hd,
                               scale=0.125, f16=int(f16), scratch=0, max_vis=max(vis), outq=d_outq.ptr)
    need = H.lib().axon_hip_attention_scratch_floats(C.byref(args), C.c_size_t(n))
    scratch = H.DeviceBuffer(max(need, 1) * 4)
    args.scratch = scratch.ptr if need else 0
    H.check(H.lib().axon_hip_attention_rows(C.byref(args), C.c_size_t(n)), "attention_rows")
    got = d_out.download(np.float32).reshape(n, n_head, hd)
    got_q = d_outq.download(np.uint8, n * nbq * 34).reshape(n, nbq * 34)
    want = np.zeros_like(got)
    for i in (0, m + 1, m + 2):
        s, L = seq_of[i], vis[i]
        want[i] = o.attention_kv_heads(q[i].reshape(1, n_head, hd), pool[s, 0, :L].copy(), pool[s, 1, :L].copy(), 1,
                                       L - 1, n_head, n_kv, hd, 0.125, 0, n_head, f16=f16)[0]
    L = n_past + m
    want[1:m + 1] = o.attention_kv_heads(q[1:m + 1].reshape(m, n_head, hd), pool[1, 0, :L].copy(),
                                         pool[1, 1, :L].copy(), m, n_past, n_head, n_kv, hd, 0.125, 0, n_head, f16=f16)
    for i in range(n):
        assert np.array_equal(got[i], want[i]), i
        assert np.array_equal(got_q[i], o.quantize_row_q8_0(want[i].ravel()).view(np.uint8).ravel()), i
