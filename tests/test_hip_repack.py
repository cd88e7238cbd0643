"""The one-time repack of Q6_K weights at upload (axon_hip_q6k_repack) and the matmul over the
repacked planes (axon_hip_matmul_q6_k_planar): the step before the path, turning the GGUF blocks
(BlockQ6_K, src/core/dtype.h; dequantize_block_q6_k, src/core/dtype.cpp:313-336) into 16-byte
aligned planes for the device.

* The planes are checked against the native block bytes by dequantization: a NumPy dequantizer
  that reads the documented planar layout directly (13 slices [rows][16 bytes] per super-block
  column, then the d plane) gives the oracle's dequantization of the native blocks, float for
  float; the oracle's dequantizer is pinned to the reference's by its fixture.
* The planar matmul equals the oracle's matmul_q6_k bit for bit (one row and several, strided
  outputs; each of the three one-row kernels forced in turn), and the native stream kernel on
  the Llama-3 output shape.
* A model's logits are the same with and without the repack."""
from dataclasses import replace

import numpy as np
import pytest

from helpers import Q6_K
from tables import CTable, HipTable, dequantize, random_floats, random_weights

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def H():
    HipTable()
    import axon_hip
    import ctypes as C
    axon_hip.lib().axon_hip_q6k_planar_bytes.restype = C.c_size_t
    return axon_hip


@pytest.fixture(scope="module")
def o():
    return CTable("oracle")


def q6k_weights(n_out, n_in, seed):
    w = random_weights("q6_k", n_out, n_in, seed)
    rng = np.random.default_rng(seed + 1)
    w["d"] = rng.uniform(1e-4, 4e-3, len(w)).astype(np.float16).view(np.uint16)  # a scale per block
    return w


def repack(H, w, n_out, n_in, native_offset=0):
    import ctypes as C
    nbytes = H.lib().axon_hip_q6k_planar_bytes(C.c_size_t(n_out), C.c_size_t(n_in))
    src = H.DeviceBuffer(w.nbytes + native_offset)
    src.upload(w.view(np.uint8), native_offset)
    dst = H.DeviceBuffer(nbytes)
    H.call("q6k_repack", src.at(native_offset), n_out, n_in, dst)
    return dst, nbytes


def dequantize_planar(planar: np.ndarray, n_out: int, n_in: int) -> np.ndarray:
    """The planar layout read back as weights: per column, slices 0-7 are ql, 8-11 qh, 12 the
    int8 scales, then the d plane; values d * scale * (q - 32) in float."""
    nsb = n_in // 256
    col = 208 * n_out + ((2 * n_out + 15) // 16) * 16
    out = np.zeros((n_out, n_in), np.float32)
    for c in range(nsb):
        reg = planar[c * col:(c + 1) * col]
        sl = reg[:208 * n_out].reshape(13, n_out, 16)
        ql = sl[0:8].transpose(1, 0, 2).reshape(n_out, 128)
        qh = sl[8:12].transpose(1, 0, 2).reshape(n_out, 64)
        sc = sl[12].view(np.int8).astype(np.float32)
        d = reg[208 * n_out:208 * n_out + 2 * n_out].view(np.float16).astype(np.float32)
        y = out[:, 256 * c:256 * (c + 1)]
        for n in range(2):
            lq, hq, s = ql[:, 64 * n:64 * n + 64], qh[:, 32 * n:32 * n + 32], sc[:, 8 * n:8 * n + 8]
            l = np.arange(32)
            iss = l // 16
            parts = [((lq[:, l] & 15) | ((hq[:, l] & 3) << 4), 0), ((lq[:, l + 32] & 15) | (((hq[:, l] >> 2) & 3) << 4), 2),
                     ((lq[:, l] >> 4) | (((hq[:, l] >> 4) & 3) << 4), 4), ((lq[:, l + 32] >> 4) | (((hq[:, l] >> 6) & 3) << 4), 6)]
            for k, (q, so) in enumerate(parts):
                ds = d[:, None] * s[:, iss + so]
                y[:, 128 * n + 32 * k + l] = ds * (q.astype(np.int32) - 32).astype(np.float32)
    return out


@pytest.mark.parametrize("n_out, n_in", [(8, 256), (13, 512), (1000, 2048), (77, 4096)])
def test_repack_dequantizes_as_the_native_blocks(H, n_out, n_in):
    w = q6k_weights(n_out, n_in, n_out + n_in)
    for off in (0, 2):  # native rows at a 2-byte (not 4-byte) boundary too
        dst, nbytes = repack(H, w, n_out, n_in, off)
        planar = dst.download(np.uint8, nbytes)
        got = dequantize_planar(planar, n_out, n_in)
        want = dequantize("q6_k", w, n_out, n_in)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("n_out, n_in", [(13, 256), (1000, 2048), (4096, 4096), (300, 8192)])
@pytest.mark.parametrize("n_rows", [1, 3, 4, 6, 9])
def test_planar_matmul_bit_exact(H, o, n_out, n_in, n_rows):
    w = q6k_weights(n_out, n_in, 3 * n_out + n_rows)
    x = random_floats(n_rows * n_in, n_in + n_rows)
    dst, _ = repack(H, w, n_out, n_in)
    stride = n_out + 1 if n_rows > 1 else n_out
    dx = H.DeviceBuffer.of(x)
    dy = H.DeviceBuffer.of(np.full(n_rows * stride, np.float32(-7.25), np.float32))
    H.call("matmul_q6_k_planar", dst, dx, dy, n_rows, n_out, n_in, stride)
    got = dy.download(np.float32, n_rows * stride)
    want = o.matmul("q6_k", w, x, n_out, n_in, n_rows=n_rows, y_stride=stride)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("path", [1, 2, 3])
@pytest.mark.parametrize("n_out, n_in", [(13, 256), (64, 512), (1000, 2048), (300, 8192), (77, 14336),
                                         (4097, 4096), (9000, 2048), (70, 40960)])
def test_one_row_kernels_bit_exact(H, o, path, n_out, n_in):
    """Each one-row kernel (axon_hip_q6k_force_path: one lane per row; products then chains,
    whose rows per workgroup shrink as n_in grows and which 40960 columns do not fit; the
    streamed ring, 64 rows per workgroup with a partial last one) against the oracle, bit for bit."""
    import ctypes as C
    w = q6k_weights(n_out, n_in, 11 * n_out + n_in)
    x = random_floats(n_in, n_in + 3 * path)
    dst, _ = repack(H, w, n_out, n_in)
    dx = H.DeviceBuffer.of(x)
    dy = H.DeviceBuffer.of(np.full(n_out + 1, np.float32(-7.25), np.float32))
    H.check(H.lib().axon_hip_q6k_force_path(C.c_int(path)), "q6k_force_path")
    try:
        H.call("matmul_q6_k_planar", dst, dx, dy, 1, n_out, n_in, n_out)
    finally:
        H.check(H.lib().axon_hip_q6k_force_path(C.c_int(0)), "q6k_force_path")
    got = dy.download(np.float32, n_out + 1)
    want = o.matmul("q6_k", w, x, n_out, n_in, n_rows=1, y_stride=n_out)
    assert np.array_equal(got[:n_out].view(np.uint32), want.view(np.uint32))
    assert got[n_out] == np.float32(-7.25)  # nothing written past the last row


def greedy_id(y):
    """std::ranges::max_element with NaN skipped, a NaN first value selecting 0 (sampler.cpp:100-102)."""
    if np.isnan(y[0]) or np.isnan(y).all():
        return 0
    return int(np.nanargmax(y))


@pytest.mark.parametrize("n_out, n_in, plant", [(1, 256, None), (7, 256, "tie"), (65, 512, "tie"), (300, 2048, "nan"),
                                                (16383, 256, "tie"), (65536, 256, None), (70001, 512, "tie")])
def test_planar_argmax_keys_and_embedding(H, o, n_out, n_in, plant):
    """axon_hip_matmul_q6_k_planar_argmax (the generate loop's output matmul): y bit for bit as
    matmul_q6_k_planar, and axon_hip_argmax_embed over its keys picks argmax_rows' id (ties to
    the first: a copy of the best row's blocks planted before and after it; a NaN first logit
    selects 0) and writes that row of the embedding table as embedding_rows does, for Q6_K, Q4_0
    and F32 tables. Workgroups of 64 rows (under 65536 outputs) and of 256 both occur."""
    import ctypes as C
    L = H.lib()
    L.axon_hip_q6k_argmax_parts.restype = C.c_size_t
    nsb = n_in // 256
    w = q6k_weights(n_out, n_in, 3 * n_out + n_in)
    x = random_floats(n_in, n_in + n_out)
    want_y = o.matmul("q6_k", w, x, n_out, n_in, n_rows=1, y_stride=n_out)
    if plant == "tie":
        j = int(np.argmax(want_y))
        for r in (j - 2, j + 3):
            if 0 <= r < n_out:
                w[r * nsb:(r + 1) * nsb] = w[j * nsb:(j + 1) * nsb]
    elif plant == "nan":
        w["d"][0:nsb] = 0x7e00  # row 0's scale: a NaN logit first
    dst, _ = repack(H, w, n_out, n_in)
    dx = H.DeviceBuffer.of(x)
    parts = L.axon_hip_q6k_argmax_parts(C.c_size_t(n_out))
    assert parts == -(-n_out // (256 if -(-n_out // 256) >= 256 else 64))
    keys = H.DeviceBuffer.of(np.full(parts + 1, 0x5a5a5a5a5a5a5a5a, np.uint64))
    y = H.DeviceBuffer.of(np.full(n_out + 1, np.float32(-7.25), np.float32))
    with pytest.raises(H.HipError, match="key words"):
        H.check(L.axon_hip_matmul_q6_k_planar_argmax(C.c_void_p(dst.ptr), C.c_void_p(dx.ptr), C.c_void_p(y.ptr),
                                                     C.c_size_t(n_out), C.c_size_t(n_in), C.c_void_p(keys.ptr),
                                                     C.c_size_t(parts - 1)), "planar_argmax")
    H.check(L.axon_hip_matmul_q6_k_planar_argmax(C.c_void_p(dst.ptr), C.c_void_p(dx.ptr), C.c_void_p(y.ptr),
                                                 C.c_size_t(n_out), C.c_size_t(n_in), C.c_void_p(keys.ptr),
                                                 C.c_size_t(parts)), "planar_argmax")
    got_y = y.download(np.float32, n_out + 1)
    assert got_y[n_out] == np.float32(-7.25)
    ref = H.DeviceBuffer(4 * n_out)
    H.call("matmul_q6_k_planar", dst, dx, ref, 1, n_out, n_in, n_out)
    assert np.array_equal(got_y[:n_out].view(np.uint32), ref.download(np.uint32, n_out))
    assert keys.download(np.uint64, parts + 1)[parts] == 0x5a5a5a5a5a5a5a5a  # no key past the count
    want_id = greedy_id(got_y[:n_out])
    if plant == "nan":
        assert want_id == 0 and np.isnan(got_y[0])
    if plant == "tie" and n_out > 2:
        j = int(np.argmax(want_y))
        assert want_id == (j - 2 if j >= 2 else j)
    scratch = H.DeviceBuffer(8 * 64)
    amax = H.DeviceBuffer(4)
    H.check(L.axon_hip_argmax_rows(C.c_void_p(y.ptr), C.c_size_t(n_out), C.c_size_t(1), C.c_size_t(n_out),
                                   C.c_void_p(scratch.ptr), C.c_void_p(amax.ptr)), "argmax_rows")
    assert int(amax.download(np.int32, 1)[0]) == want_id
    n_emb = 512 if n_out < 20000 else 256
    for kind, tid in (("q6_k", 14), ("q4_0", 2), ("f32", 0)):
        rows = max(n_out, 2)
        table = (random_floats(rows * n_emb, 5) if kind == "f32"
                 else random_weights(kind, rows, n_emb, 9 + n_out))
        dtab = H.DeviceBuffer.of(table)
        emb = H.DeviceBuffer.of(np.full(n_emb, np.float32(3.5), np.float32))
        out_id = H.DeviceBuffer.of(np.array([-5], np.int32))
        H.check(L.axon_hip_argmax_embed(C.c_void_p(y.ptr), C.c_void_p(keys.ptr), C.c_size_t(parts),
                                        C.c_void_p(out_id.ptr), C.c_int(tid), C.c_void_p(dtab.ptr), C.c_size_t(rows),
                                        C.c_size_t(n_emb), C.c_void_p(emb.ptr)), "argmax_embed")
        assert int(out_id.download(np.int32, 1)[0]) == want_id, kind
        ids = H.DeviceBuffer.of(np.array([want_id], np.int32))
        want_emb = H.DeviceBuffer(4 * n_emb)
        H.check(L.axon_hip_embedding_rows(C.c_int(tid), C.c_void_p(dtab.ptr), C.c_size_t(n_emb), C.c_void_p(ids.ptr),
                                          C.c_size_t(1), C.c_void_p(want_emb.ptr)), "embedding_rows")
        assert np.array_equal(emb.download(np.uint32, n_emb), want_emb.download(np.uint32, n_emb)), kind


def test_force_path_bounds(H):
    import ctypes as C
    with pytest.raises(H.HipError, match="0-3"):
        H.check(H.lib().axon_hip_q6k_force_path(C.c_int(4)), "q6k_force_path")


def test_planar_matmul_equals_the_stream_kernel_on_the_output_shape(H):
    n_out, n_in = 128256, 2048
    w = q6k_weights(n_out, n_in, 5)
    dst, _ = repack(H, w, n_out, n_in)
    dw = H.DeviceBuffer.of(w)
    for n_rows in (1, 3, 4, 5, 6, 7, 12, 20, 28, 32):
        x = random_floats(n_rows * n_in, 40 + n_rows)
        dx = H.DeviceBuffer.of(x)
        a = H.DeviceBuffer(4 * n_rows * n_out)
        b = H.DeviceBuffer(4 * n_rows * n_out)
        H.call("matmul_q6_k_planar", dst, dx, a, n_rows, n_out, n_in, n_out)
        H.call("matmul_q6_k_rows", dw, dx, b, n_rows, n_out, n_in, n_out)
        assert np.array_equal(a.download(np.uint32, n_rows * n_out), b.download(np.uint32, n_rows * n_out))


@pytest.mark.parametrize("n_rows", [8, 16, 21, 32])
def test_native_rows_bit_exact(H, o, n_rows):
    """matmul_q6_k_rows over the GGUF blocks with many activation rows (launches of up to four,
    then the rest), strided outputs, against the oracle."""
    n_out, n_in = 300, 2048
    w = q6k_weights(n_out, n_in, 7 * n_rows)
    x = random_floats(n_rows * n_in, 90 + n_rows)
    stride = n_out + 3
    dw = H.DeviceBuffer.of(w)
    dx = H.DeviceBuffer.of(x)
    dy = H.DeviceBuffer.of(np.full(n_rows * stride, np.float32(-7.25), np.float32))
    H.call("matmul_q6_k_rows", dw, dx, dy, n_rows, n_out, n_in, stride)
    got = dy.download(np.float32, n_rows * stride)
    want = o.matmul("q6_k", w, x, n_out, n_in, n_rows=n_rows, y_stride=stride)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_planar_bounds(H):
    import ctypes as C
    assert H.lib().axon_hip_q6k_planar_bytes(C.c_size_t(10), C.c_size_t(300)) == 0
    assert H.lib().axon_hip_q6k_planar_bytes(C.c_size_t(8), C.c_size_t(512)) == 2 * 8 * 210
    assert H.lib().axon_hip_q6k_planar_bytes(C.c_size_t(9), C.c_size_t(256)) == 208 * 9 + 32
    buf = H.DeviceBuffer(4096)
    with pytest.raises(H.HipError, match="multiple of 256"):
        H.call("q6k_repack", buf, 4, 300, buf)
    with pytest.raises(H.HipError, match="aligned"):
        H.call("q6k_repack", buf.at(1), 1, 256, buf)
    with pytest.raises(H.HipError, match="aligned"):
        H.call("matmul_q6_k_planar", buf.at(8), buf, buf, 1, 1, 256, 1)
    with pytest.raises(H.HipError, match="positive multiple of 256"):  # no super-block to read
        H.call("matmul_q6_k_planar", buf, buf, buf, 1, 4, 0, 4)
    with pytest.raises(H.HipError, match="positive multiple of 256"):
        H.call("matmul_q6_k_rows", buf, buf, buf, 1, 4, 0, 4)


def test_model_logits_unchanged_by_the_repack(H, tmp_path_factory):
    """The config-4 shape (tied Q6_K output) at 2 layers and a 2048-token vocabulary: the same
    logits bit for bit with and without the repacked output matrix, for a prefill and a batch."""
    import synth
    spec = replace(synth.CONFIGS["c4"], name="t-c4-repack-2l", n_layer=2, n_vocab=2048, seed=17)
    path = synth.cached_model(spec, tmp_path_factory.mktemp("models"))
    toks = np.random.default_rng(3).integers(0, 2048, 21).astype(np.int32)
    out = []
    for repack_on in (True, False):
        m = H.Model(path, max_seq=32, max_ctx=64, max_batch=3, max_caches=4, repack=repack_on)
        c = m.new_cache()
        a = m.forward_prefill(c, toks[:13])
        cs = [c, m.new_cache(), m.new_cache()]
        m.forward_prefill(cs[1], toks[13:17])
        m.forward_prefill(cs[2], toks[17:18])
        b = m.forward_batch(cs, toks[18:21])
        out.append((a, b, m.info.device_bytes))
        m.close()
    assert np.array_equal(out[0][0], out[1][0]) and np.array_equal(out[0][1], out[1][1])
    assert out[0][2] - out[1][2] == 2048 * 2048 // 256 * 210
