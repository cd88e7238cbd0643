"""The allocation-free greedy choice (axon_hip_argmax_rows_noalloc) against the workspace entry
(axon_hip_argmax_rows) through the C ABI: the same ids, bit for bit, on two calls in a row (the
second with fewer rows and a shorter vocabulary, over the scratch the first call left behind),
and a refused call beyond the fixed scratch's row bound.

Selection is index work, so the bar is exact ids. Both entries are also checked against numpy's
first-maximum argmax, which is max_element's choice on NaN-free rows (the oracle sampler's tests
pin that equivalence); rows with NaN are compared between the two entries only."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

MAX_ROWS = 512  # AXON_HIP_ARGMAX_NOALLOC_MAX_ROWS


@pytest.fixture(scope="module")
def H():
    import axon_hip
    axon_hip.init(0)
    axon_hip.lib().axon_hip_argmax_scratch_words.restype = C.c_size_t
    return axon_hip


def logits(n, n_rows, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n_rows, n)).astype(np.float32)
    for r in range(0, n_rows, 5):  # the same maximum twice: the first must win
        j0, j1 = sorted(rng.choice(n, 2, replace=False))
        x[r, j0] = x[r, j1] = np.float32(7.0)
    return x


def with_workspace(H, dx, n, n_rows):
    words = H.lib().axon_hip_argmax_scratch_words(C.c_size_t(n_rows))
    scratch = H.DeviceBuffer(8 * words)
    out = H.DeviceBuffer(4 * n_rows)
    out.upload(np.full(n_rows, -7, np.int32))
    H.call("argmax_rows", dx, n, n_rows, n, scratch, out)
    return out.download(np.int32, n_rows)


def without_allocation(H, dx, n, n_rows):
    out = H.DeviceBuffer(4 * n_rows)
    out.upload(np.full(n_rows, -9, np.int32))
    H.call("argmax_rows_noalloc", dx, n, n_rows, n, out)
    return out.download(np.int32, n_rows)


def test_noalloc_argmax_equals_workspace_argmax_on_two_calls(H):
    cases = [(128256, 300, 1), (1000, 7, 2)]  # the second call smaller than the first
    for n, n_rows, seed in cases:
        x = logits(n, n_rows, seed)
        dx = H.DeviceBuffer.of(x)
        got = without_allocation(H, dx, n, n_rows)
        want = with_workspace(H, dx, n, n_rows)
        assert np.array_equal(got, want), (n, n_rows)
        assert np.array_equal(got, np.argmax(x, axis=1).astype(np.int32)), (n, n_rows)


def test_noalloc_argmax_at_the_row_bound_and_beyond(H):
    n = 4097
    x = logits(n, MAX_ROWS, 3)
    x[1, 0] = np.float32("nan")  # a NaN first element selects index 0 on both entries
    dx = H.DeviceBuffer.of(x)
    got = without_allocation(H, dx, n, MAX_ROWS)
    assert np.array_equal(got, with_workspace(H, dx, n, MAX_ROWS))
    assert got[1] == 0
    out = H.DeviceBuffer(4 * (MAX_ROWS + 1))
    big = H.DeviceBuffer(4 * n * (MAX_ROWS + 1))
    with pytest.raises(H.HipError, match="exceed the fixed scratch"):
        H.call("argmax_rows_noalloc", big, n, MAX_ROWS + 1, n, out)
