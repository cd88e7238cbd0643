"""Graph capture on the library stream (axon_hip_graph_begin / end / launch / destroy): the Q8_0
quantization and a Q4_0 matvec captured into a graph replay to the eager results, three times,
with other eager work and synchronizations between the replays; and axon_hip_memset refuses while
a capture is open (a memset node is not replayed reliably on this platform, and the entry's
synchronize is illegal under capture)."""
import ctypes as C

import numpy as np
import pytest

from tables import random_floats, random_weights

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def H():
    import axon_hip
    axon_hip.init(0)
    return axon_hip


def test_captured_entries_replay_to_the_eager_result(H):
    n_rows, n_in, n_out = 3, 2048, 512
    x = random_floats(n_rows * n_in, 5, 3.0)
    w = random_weights("q4_0", n_out, n_in, 6)
    dx, dw = H.DeviceBuffer.of(x), H.DeviceBuffer.of(w)
    xq = H.DeviceBuffer(n_rows * n_in // 32 * 34)
    y = H.DeviceBuffer(n_rows * n_out * 4)
    H.call("quantize_rows_q8_0", dx, xq, n_in, n_rows, n_in)
    H.call("matmul_q4_0_q8_rows", dw, xq, y, n_rows, n_out, n_in, n_out)
    H.synchronize()
    want = y.download(np.float32)

    xq2, y2 = H.DeviceBuffer(xq.nbytes), H.DeviceBuffer(y.nbytes)
    H.check(H.lib().axon_hip_graph_begin(), "graph_begin")
    H.call("quantize_rows_q8_0", dx, xq2, n_in, n_rows, n_in)
    H.call("matmul_q4_0_q8_rows", dw, xq2, y2, n_rows, n_out, n_in, n_out)
    g = C.c_void_p(0)
    H.check(H.lib().axon_hip_graph_end(C.byref(g)), "graph_end")
    other = H.DeviceBuffer.of(random_floats(n_rows * n_in, 7, 1.0))
    try:
        for replay in range(3):
            y2.upload(np.full(n_rows * n_out, np.float32(np.nan), np.float32))
            H.check(H.lib().axon_hip_graph_launch(g), "graph_launch")
            H.synchronize()
            assert np.array_equal(y2.download(np.float32), want), replay
            # eager work between replays, on other buffers
            H.call("quantize_rows_q8_0", other, xq, n_in, n_rows, n_in)
            H.call("matmul_q4_0_q8_rows", dw, xq, y, n_rows, n_out, n_in, n_out)
            H.synchronize()
    finally:
        H.lib().axon_hip_graph_destroy(g)


def test_memset_is_refused_while_a_capture_is_open(H):
    buf = H.DeviceBuffer(256)
    acc = H.DeviceBuffer.of(np.ones(16, np.float32))
    H.check(H.lib().axon_hip_graph_begin(), "graph_begin")
    try:
        H.call("add", acc, acc, 16)  # a captured kernel, so the graph is not empty
        with pytest.raises(H.HipError, match="graph capture"):
            buf.fill(0)
    finally:
        g = C.c_void_p(0)
        H.check(H.lib().axon_hip_graph_end(C.byref(g)), "graph_end")
        H.lib().axon_hip_graph_destroy(g)
    buf.fill(0)  # outside a capture it runs
    assert not buf.download(np.uint8).any()
