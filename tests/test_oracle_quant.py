"""Pins the oracle's conversions, block formats, Q8_0 quantizer and integer-dot matmuls
against the reference's golden fixtures (tests/golden/quant, written by the gguf package's
ggml-exact quantizer) and against closed forms. Mirrors tests/unit/test_dtype_quant.cpp and
tests/unit/test_kernels_quant.cpp of the reference."""
import numpy as np
import pytest

from helpers import (BF16, F16, F32, Q4_0, Q4_0_ID, Q4_1, Q4_1_ID, Q6_K, Q6_K_ID, Q8_0, Q8_0_ID, call,
                     golden, golden_blocks, oracle)


def fp16_table(lib):
    return np.array([lib.ora_fp16_to_fp32(h) for h in range(65536)], dtype=np.float32)


def test_fp16_widening_is_exact_for_every_pattern():
    # numpy's float16 -> float32 is exact, including subnormals and inf; nan stays nan.
    lib = oracle()
    got = fp16_table(lib)
    want = np.arange(65536, dtype=np.uint16).view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_fp16_narrowing_rounds_to_nearest_even():
    lib = oracle()
    rng = np.random.default_rng(1)
    # Normal range, subnormal halves, ties, overflow and underflow.
    xs = np.concatenate([
        rng.normal(0, 1, 20000), rng.uniform(-7e4, 7e4, 5000), rng.uniform(-1e-4, 1e-4, 5000),
        rng.uniform(-1e-7, 1e-7, 2000), [65504.0, 65519.9, 65520.0, 1e6, -1e6, 0.0, -0.0, 2**-24, 2**-25,
                                        3 * 2**-26, 1.0 + 2**-11, 1.0 + 3 * 2**-11],
    ]).astype(np.float32)
    got = np.array([lib.ora_fp32_to_fp16(float(x)) for x in xs], dtype=np.uint16)
    want = xs.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def test_bf16_round_trip():
    lib = oracle()
    rng = np.random.default_rng(2)
    xs = rng.normal(0, 10, 5000).astype(np.float32)
    got = np.array([lib.ora_fp32_to_bf16(float(x)) for x in xs], dtype=np.uint16)
    # Round to nearest even on the top 16 bits, computed independently in integers.
    u = xs.view(np.uint32).astype(np.uint64)
    want = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    assert np.array_equal(got, want)
    back = np.array([lib.ora_bf16_to_fp32(int(h)) for h in got], dtype=np.float32)
    assert np.array_equal(back.view(np.uint32), got.astype(np.uint32) << 16)


@pytest.mark.parametrize("name,dt,fn,qk", [
    ("q8_0", Q8_0, "ora_dequantize_block_q8_0", 32),
    ("q4_0", Q4_0, "ora_dequantize_block_q4_0", 32),
    ("q4_1", Q4_1, "ora_dequantize_block_q4_1", 32),
    ("q6_k", Q6_K, "ora_dequantize_block_q6_k", 256),
])
def test_dequantize_matches_gguf_package(name, dt, fn, qk):
    lib = oracle()
    blocks = golden_blocks(f"quant/row.{name}.bin", dt)
    want = golden(f"quant/row.{name}.dequant.axt")
    got = np.zeros(len(blocks) * qk, dtype=np.float32)
    for b in range(len(blocks)):
        one = blocks[b:b + 1].copy()
        call(lib, fn, one, got[b * qk:(b + 1) * qk])
    assert np.array_equal(got, want)


@pytest.mark.parametrize("base", ["row", "act"])
def test_quantize_row_q8_0_is_byte_exact(base):
    lib = oracle()
    x = golden(f"quant/{base}.f32.axt")
    want = (golden_blocks(f"quant/{base}.q8_0.bin", Q8_0))
    got = np.zeros(len(x) // 32, dtype=Q8_0)
    call(lib, "ora_quantize_row_q8_0", x, got, len(x))
    assert got.tobytes() == want.tobytes()


def test_quantize_round_trip_within_a_rounded_quantum():
    # tests/unit/test_dtype_quant.cpp:76-99
    lib = oracle()
    x = ((np.arange(64) - 31) * np.float32(0.37)).astype(np.float32)
    q = np.zeros(2, dtype=Q8_0)
    call(lib, "ora_quantize_row_q8_0", x, q, 64)
    back = np.zeros(64, dtype=np.float32)
    for b in range(2):
        call(lib, "ora_dequantize_block_q8_0", q[b:b + 1].copy(), back[b * 32:(b + 1) * 32])
    d = np.array([lib.ora_fp16_to_fp32(int(q[i // 32]["d"])) for i in range(64)], dtype=np.float32)
    assert np.all(np.abs(back - x) <= d * 0.57 + 1e-6)
    assert np.any(np.abs(q["qs"]) == 127)


@pytest.mark.parametrize("name,dt,entry", [
    ("matmul_q8_0", Q8_0, "ora_matmul_q8_0_q8"),
    ("matmul_q4_0", Q4_0, "ora_matmul_q4_0_q8"),
    ("matmul_q4_1", Q4_1, "ora_matmul_q4_1_q8"),
])
def test_integer_matmul_matches_float64_int_dot(name, dt, entry):
    # tests/unit/test_kernels_quant.cpp:50-84, 101-134: 1e-5 against the float64 reference.
    lib = oracle()
    w = golden_blocks(f"quant/{name}.w.bin", dt)
    xq = golden_blocks(f"quant/{name}.xq.bin", Q8_0)
    want = golden(f"quant/{name}.yq.axt")
    n_out, n_in = 7, 96
    y = np.zeros(n_out, dtype=np.float32)
    call(lib, entry, w, xq, y, n_out, n_in)
    assert np.max(np.abs(y - want)) < 1e-5
    # Q8_0 quantization of x reproduces the fixture's activation blocks.
    x = golden(f"quant/{name}.x.axt")
    mine = np.zeros(n_in // 32, dtype=Q8_0)
    call(lib, "ora_quantize_row_q8_0", x, mine, n_in)
    assert mine.tobytes() == xq.tobytes()
    # Rows variant over three rows.
    xs = golden(f"quant/{name}.xs.axt")
    xsq = np.zeros(3 * n_in // 32, dtype=Q8_0)
    for r in range(3):
        part = np.zeros(n_in // 32, dtype=Q8_0)
        call(lib, "ora_quantize_row_q8_0", np.ascontiguousarray(xs[r]), part, n_in)
        xsq[r * 3:(r + 1) * 3] = part
    ys = np.zeros((3, n_out), dtype=np.float32)
    call(lib, entry + "_rows", w, xsq, ys, 3, n_out, n_in, n_out)
    assert np.max(np.abs(ys - golden(f"quant/{name}.ysq.axt"))) < 1e-5


@pytest.mark.parametrize("name,dt,entry", [
    ("matmul_q8_0", Q8_0, "ora_matmul_q8_0"),
    ("matmul_q4_0", Q4_0, "ora_matmul_q4_0"),
    ("matmul_q4_1", Q4_1, "ora_matmul_q4_1"),
])
def test_float_activation_matmul_matches_dequantized_float64(name, dt, entry):
    lib = oracle()
    w = golden_blocks(f"quant/{name}.w.bin", dt)
    x = golden(f"quant/{name}.x.axt")
    y = np.zeros(7, dtype=np.float32)
    call(lib, entry, w, x, y, 7, 96)
    assert np.max(np.abs(y - golden(f"quant/{name}.y.axt"))) < 1e-5
    xs = golden(f"quant/{name}.xs.axt")
    ys = np.zeros((3, 7), dtype=np.float32)
    call(lib, entry + "_rows", w, xs, ys, 3, 7, 96, 7)
    assert np.max(np.abs(ys - golden(f"quant/{name}.ys.axt"))) < 1e-5


def test_q6_k_matmul_matches_fixture():
    # tests/unit/test_kernels_quant.cpp:86-99: 1e-3 against the float64 reference.
    lib = oracle()
    w = golden_blocks("quant/matmul_q6_k.w.bin", Q6_K)
    x = golden("quant/matmul_q6_k.x.axt")
    y = np.zeros(5, dtype=np.float32)
    call(lib, "ora_matmul_q6_k", w, x, y, 5, 256)
    assert np.max(np.abs(y - golden("quant/matmul_q6_k.y.axt"))) < 1e-3
    xs = golden("quant/matmul_q6_k.xs.axt")
    ys = np.zeros((3, 5), dtype=np.float32)
    call(lib, "ora_matmul_q6_k_rows", w, xs, ys, 3, 5, 256, 5)
    assert np.max(np.abs(ys - golden("quant/matmul_q6_k.ys.axt"))) < 1e-3


def test_single_block_dot_closed_form():
    # tests/unit/test_kernels_quant.cpp:136-152: one block of known integers, exact.
    lib = oracle()
    w = np.zeros(1, dtype=Q8_0)
    x = np.zeros(1, dtype=Q8_0)
    w["d"] = np.float16(0.5).view(np.uint16)
    x["d"] = np.float16(0.25).view(np.uint16)
    w["qs"][0] = np.arange(32) - 16
    x["qs"][0] = 3 - (np.arange(32) % 7)
    want = float(np.dot((np.arange(32) - 16), 3 - (np.arange(32) % 7))) * 0.5 * 0.25
    y = np.zeros(1, dtype=np.float32)
    call(lib, "ora_matmul_q8_0_q8", w, x, y, 1, 32)
    assert y[0] == np.float32(want)
    # The same integers as Q4_0 nibbles (w - 8 in [-8, 7]).
    w4 = np.zeros(1, dtype=Q4_0)
    w4["d"] = w["d"]
    ints = (np.arange(32) % 16)  # nibble values; weights are nibble - 8
    w4["qs"][0] = (ints[:16] | (ints[16:] << 4)).astype(np.uint8)
    want4 = float(np.dot(ints - 8, 3 - (np.arange(32) % 7))) * 0.5 * 0.25
    call(lib, "ora_matmul_q4_0_q8", w4, x, y, 1, 32)
    assert y[0] == np.float32(want4)


@pytest.mark.parametrize("name,dt,type_id,qk", [
    ("q8_0", Q8_0, Q8_0_ID, 32), ("q4_0", Q4_0, Q4_0_ID, 32), ("q4_1", Q4_1, Q4_1_ID, 32),
    ("q6_k", Q6_K, Q6_K_ID, 256),
])
def test_quantized_embedding_rows_exact(name, dt, type_id, qk):
    # tests/unit/test_kernels_quant.cpp:154-175
    lib = oracle()
    table = golden_blocks(f"quant/embedding_{name}.table.bin", dt)
    index = golden(f"quant/embedding_{name}.index.axt")
    want = golden(f"quant/embedding_{name}.rows.axt")
    n = want.shape[1]
    for i, idx in enumerate(index):
        out = np.zeros(n, dtype=np.float32)
        call(lib, "ora_embedding_row", type_id, table, n, int(idx), out)
        assert np.array_equal(out, want[i])


@pytest.mark.parametrize("name,type_id", [("f32", F32), ("f16", F16), ("bf16", BF16)])
def test_float_embedding_rows_exact(name, type_id):
    # tests/unit/test_kernels_embedding.cpp:12-37
    lib = oracle()
    table = golden(f"kernels/embedding_{name}.table.axt")
    index = golden(f"kernels/embedding_{name}.index.axt")
    want = golden(f"kernels/embedding_{name}.rows.axt")
    n = table.shape[1]
    for i, idx in enumerate(index):
        out = np.zeros(n, dtype=np.float32)
        call(lib, "ora_embedding_row", type_id, np.ascontiguousarray(table), n, int(idx), out)
        assert np.array_equal(out, want[i].astype(np.float32) if want.dtype == np.float32 else
                              (want[i].view(np.float16).astype(np.float32) if name == "f16" else
                               (want[i].astype(np.uint32) << 16).view(np.float32)))


def test_block_sums_hook_matches_closed_form():
    lib = oracle()
    rng = np.random.default_rng(5)
    nb = 9
    w = np.zeros(nb, dtype=Q4_1)
    w["qs"] = rng.integers(0, 256, (nb, 16), dtype=np.uint8)
    x = np.zeros(nb, dtype=Q8_0)
    x["qs"] = rng.integers(-127, 128, (nb, 32), dtype=np.int8)
    si = np.zeros(nb, dtype=np.int32)
    sx = np.zeros(nb, dtype=np.int32)
    call(lib, "ora_block_sums", Q4_1_ID, w, x, nb, si, sx)
    nib = np.concatenate([w["qs"] & 0x0F, w["qs"] >> 4], axis=1).astype(np.int64)
    assert np.array_equal(si, (nib * x["qs"].astype(np.int64)).sum(1))
    assert np.array_equal(sx, x["qs"].astype(np.int64).sum(1))
