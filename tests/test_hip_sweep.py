"""The BASELINE matvec/matmul sweep (configuration 2) through the table entries, bit-exact against
the oracle: (N, K) in {(2048, 2048), (8192, 2048), (2048, 8192), (128256, 2048)} x {Q4_0, Q4_1,
Q8_0, Q6_K} x M in {1, 16, 64, 512} activation rows ~N(0, 1). Integer types take Q8_0 activations
(matmul_*_q8 for one row, matmul_*_q8_rows for more; the activations' Q8_0 blocks themselves are
compared first); Q6_K takes float activations (matmul_q6_k / matmul_q6_k_rows over the GGUF blocks,
and matmul_q6_k_planar over the copy repacked at upload, which is what the model streams).

The reference measures these kernels in bench/bench_kernels.cpp:379-402 and checks its tables
against the scalar one in test_kernels_neon.cpp; this is that check at the sweep's shapes. The
device computes every output. Where M * N * K exceeds the oracle's budget, the oracle computes a
strided sample of weight rows (the first and the last included) for every activation row; outputs
depend on their own weight row and activation row only, so a sampled row is checked in full.
Weights are random blocks as the reference's cross-table tests build them (tables.random_weights).
"""
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

from helpers import Q4_0_ID, Q4_1_ID, Q6_K_ID, Q8_0_ID, row_bytes
from tables import CTable, random_weights

pytestmark = pytest.mark.gpu

SHAPES = [(2048, 2048), (8192, 2048), (2048, 8192), (128256, 2048)]
ROWS = [1, 16, 64, 512]
TYPE_ID = {"q4_0": Q4_0_ID, "q4_1": Q4_1_ID, "q8_0": Q8_0_ID, "q6_k": Q6_K_ID}
BUDGET = 1 << 29  # multiply-adds the oracle spends per (type, shape, M)


def workers():
    try:
        return max(1, min(16, len(os.sched_getaffinity(0))))
    except AttributeError:
        return 4


@pytest.fixture(scope="module")
def o():
    return CTable("oracle")


@pytest.fixture(scope="module")
def H():
    import axon_hip
    axon_hip.init(0)
    return axon_hip


def oracle_rows(o, kind, w_rows, x, xq, m, n, k):
    """The oracle's output for weight rows w_rows ([n] rows of blocks) against m activation rows,
    split over host threads by weight row (ctypes releases the interpreter lock)."""
    nw = workers()
    bounds = np.linspace(0, n, nw + 1).astype(int)

    def part(i):
        lo, hi = bounds[i], bounds[i + 1]
        if hi <= lo:
            return np.zeros((m, 0), np.float32)
        w = np.ascontiguousarray(w_rows[lo:hi])
        if kind == "q6_k":
            y = o.matmul("q6_k", w, x, hi - lo, k, n_rows=m, y_stride=hi - lo)
        else:
            y = o.matmul(f"{kind}_q8", w, xq, hi - lo, k, n_rows=m, y_stride=hi - lo)
        return y.reshape(m, hi - lo)

    with ThreadPoolExecutor(nw) as ex:
        return np.concatenate(list(ex.map(part, range(nw))), axis=1)


@pytest.mark.parametrize("n,k", SHAPES, ids=[f"{n}x{k}" for n, k in SHAPES])
@pytest.mark.parametrize("kind", list(TYPE_ID))
def test_sweep_bit_exact(H, o, kind, n, k):
    w = random_weights(kind, n, k, n + k)
    rb = row_bytes(TYPE_ID[kind], k)
    wr = w.view(np.uint8).reshape(n, rb)
    dw = H.DeviceBuffer.of(wr)
    planar = None
    if kind == "q6_k":
        import ctypes as C
        H.lib().axon_hip_q6k_planar_bytes.restype = C.c_size_t
        pb = H.lib().axon_hip_q6k_planar_bytes(C.c_size_t(n), C.c_size_t(k))
        planar = H.DeviceBuffer(pb)
        H.call("q6k_repack", dw, n, k, planar)
    for m in ROWS:
        x = np.random.default_rng(m * 7 + n).standard_normal(m * k).astype(np.float32)
        dx = H.DeviceBuffer.of(x)
        xq = None
        dxq = None
        if kind != "q6_k":
            xq = np.concatenate([o.quantize_row_q8_0(x[i * k:(i + 1) * k]) for i in range(m)])
            dxq = H.DeviceBuffer(xq.nbytes)
            H.call("quantize_rows_q8_0", dx, dxq, k, m, k)
            assert dxq.download(np.uint8, xq.nbytes).tobytes() == xq.tobytes(), (kind, n, k, m)
        y = H.DeviceBuffer(m * n * 4)
        if kind == "q6_k":
            if m == 1:
                H.call("matmul_q6_k", dw, dx, y, n, k)
            else:
                H.call("matmul_q6_k_rows", dw, dx, y, m, n, k, n)
        elif m == 1:
            H.call(f"matmul_{kind}_q8", dw, dxq, y, n, k)
        else:
            H.call(f"matmul_{kind}_q8_rows", dw, dxq, y, m, n, k, n)
        got = y.download(np.float32).reshape(m, n)
        if planar is not None:
            yp = H.DeviceBuffer(m * n * 4)
            H.call("matmul_q6_k_planar", planar, dx, yp, m, n, k, n)
            assert np.array_equal(yp.download(np.float32).reshape(m, n), got), (kind, n, k, m, "planar")
        # The oracle on every weight row, or on a strided sample of them.
        n_check = min(n, max(64, BUDGET // (m * k)))
        pick = np.unique(np.concatenate([np.linspace(0, n - 1, n_check).astype(int), [n - 1]]))
        want = oracle_rows(o, kind, wr[pick], x, xq, m, len(pick), k)
        assert np.array_equal(got[:, pick], want), (kind, n, k, m, len(pick))
