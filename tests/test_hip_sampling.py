"""The device greedy step (sampling.hip: axon_hip_repeat_penalty_rows, axon_hip_argmax_rows, and
the model's axon_model_greedy) against the oracle's sampler at temperature zero, which
tests/test_oracle_sampling.py pins to the reference's Sampler draw for draw.

Greedy selection is index work, so the bar is bit-exact: the same id for every row, and the
penalised logits bit-identical to the oracle's. Rows cover the full Llama-3 vocabulary (128256),
widths around the kernel's 64-way split (1, 63, 64, 65, 4097), ties placed across split
boundaries, NaN (first element and elsewhere), signed zeros, infinities and strided rows."""
import ctypes as C
from dataclasses import replace

import numpy as np
import pytest

from helpers import OracleModel
from tables import HipTable
from test_oracle_sampling import OracleSampler, greedy, penalize

pytestmark = pytest.mark.gpu

NAN = np.float32("nan")


@pytest.fixture(scope="module")
def H():
    HipTable()
    import axon_hip
    axon_hip.lib().axon_hip_argmax_scratch_words.restype = C.c_size_t
    return axon_hip


def device_argmax(H, x, n, n_rows, stride):
    words = H.lib().axon_hip_argmax_scratch_words(C.c_size_t(n_rows))
    dx = H.DeviceBuffer.of(np.ascontiguousarray(x, np.float32))
    scratch = H.DeviceBuffer(8 * max(words, 1))
    out = H.DeviceBuffer(4 * max(n_rows, 1))
    out.upload(np.full(max(n_rows, 1), -7, np.int32))
    H.call("argmax_rows", dx, n, n_rows, stride, scratch, out)
    return out.download(np.int32, n_rows)


def rows_with_cases(n, n_rows, seed):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((n_rows, n)).astype(np.float32)
    for r in range(n_rows):
        kind = r % 8
        if kind == 1 and n > 2:   # a tie: the same maximum at two places, the first must win
            j0, j1 = sorted(rng.choice(n, 2, replace=False))
            x[r, j0] = x[r, j1] = np.float32(9.0)
        elif kind == 2:           # NaN at the front selects 0
            x[r, 0] = NAN
        elif kind == 3 and n > 1:  # NaN elsewhere is skipped
            x[r, rng.integers(1, n, max(1, n // 7))] = NAN
        elif kind == 4:           # every value equal: index 0
            x[r, :] = np.float32(-1.5)
        elif kind == 5 and n > 1:  # -0 and +0 as the maximum
            x[r, :] = np.float32(-3.0)
            x[r, n - 1] = np.float32(0.0)
            x[r, n // 2] = np.float32(-0.0)
        elif kind == 6:           # infinities
            x[r, rng.integers(0, n)] = np.float32(np.inf)
            x[r, rng.integers(0, n)] = np.float32(-np.inf)
        elif kind == 7:           # all NaN
            x[r, :] = NAN
    return x


@pytest.mark.parametrize("n", [1, 2, 63, 64, 65, 1000, 4097, 32000, 128256])
def test_argmax_rows_match_oracle(H, n):
    n_rows = 8
    x = rows_with_cases(n, n_rows, n)
    got = device_argmax(H, x, n, n_rows, n)
    want = [greedy(x[r]) for r in range(n_rows)]
    assert got.tolist() == want


def test_argmax_ties_across_every_part_boundary(H):
    # The maximum appears at the last element of one part and the first of the next: the
    # earlier index must win whichever part reduces first.
    n = 128256
    chunk = (n + 63) // 64
    rows = []
    for b in range(1, 64, 9):
        x = np.zeros(n, np.float32)
        x[b * chunk - 1] = x[b * chunk] = np.float32(3.0)
        x[n - 1] = np.float32(3.0)
        rows.append(x)
    x = np.stack(rows)
    got = device_argmax(H, x, n, len(rows), n)
    assert got.tolist() == [greedy(r) for r in rows]


def test_argmax_strided_rows(H):
    n, stride, n_rows = 5000, 5120, 5
    x = np.random.default_rng(3).standard_normal((n_rows, stride)).astype(np.float32)
    x[:, n:] = np.float32(100.0)  # past each row's end: must not be read as part of the row
    got = device_argmax(H, x, n, n_rows, stride)
    assert got.tolist() == [int(np.argmax(x[r, :n])) for r in range(n_rows)]


def test_argmax_rejects_bad_arguments(H):
    dx = H.DeviceBuffer(64)
    s = H.DeviceBuffer(8 * 64)
    out = H.DeviceBuffer(4)
    with pytest.raises(H.HipError):
        H.call("argmax_rows", dx, 16, 1, 8, s, out)    # stride < n
    with pytest.raises(H.HipError):
        H.call("argmax_rows", dx, 0, 1, 16, s, out)    # empty rows
    with pytest.raises(H.HipError):
        H.call("argmax_rows", dx, 16, 1, 16, None, out)


def device_penalty(H, x, windows, penalty):
    n_rows, n = x.shape
    width = max(1, max(len(w) for w in windows))
    win = np.zeros((n_rows, width), np.int32)
    lens = np.zeros(n_rows, np.uint32)
    for r, w in enumerate(windows):
        win[r, :len(w)] = w
        lens[r] = len(w)
    dx = H.DeviceBuffer.of(x)
    H.call("repeat_penalty_rows", dx, n, n_rows, n, H.DeviceBuffer.of(win), H.DeviceBuffer.of(lens), width,
           float(penalty))
    return dx.download(np.float32, n_rows * n).reshape(n_rows, n)


@pytest.mark.parametrize("penalty", [1.1, 1.5, 0.8, 2.5])
def test_repeat_penalty_bit_exact(H, penalty):
    rng = np.random.default_rng(int(penalty * 10))
    n, n_rows = 32000, 6
    x = rng.standard_normal((n_rows, n)).astype(np.float32)
    x[0, :4] = [0.0, -0.0, NAN, np.inf]
    windows = [
        [0, 1, 2, 3, 0, 1, 2, 3],                                # zeros, NaN, inf, repeated ids
        rng.integers(0, n, 64).tolist(),
        rng.integers(-5, n + 5, 300).tolist(),                   # out-of-range ids are ignored
        [7] * 50,                                                # one id, many times: rescaled once
        [],
        rng.integers(0, 40, 1000).tolist(),                      # a long window with heavy repeats
    ]
    got = device_penalty(H, x, windows, penalty)
    for r in range(n_rows):
        want = penalize(x[r], windows[r], penalty, 1 << 30)
        assert np.array_equal(got[r].view(np.uint32), want.view(np.uint32)), r


# ---- the model's greedy step --------------------------------------------------------------------


def hip_model(path, **kw):
    import axon_hip as H
    return H.Model(path, **kw)


@pytest.fixture(scope="module")
def c1_model(tmp_path_factory):
    import synth
    spec = replace(synth.CONFIGS["c1"], name="t-c1-greedy-2l", n_layer=2, n_vocab=2048, seed=13)
    return synth.cached_model(spec, tmp_path_factory.mktemp("models"))


@pytest.mark.parametrize("penalty, last_n", [(1.0, 64), (1.1, 64), (1.5, 8)])
def test_model_greedy_64_steps_match_oracle_sampler(H, c1_model, penalty, last_n):
    """64 greedy steps with the device sampler (logits never leave HBM) against the oracle's
    forward pass and the oracle's sampler at temperature zero with the same penalty."""
    prompt = np.random.default_rng(7).integers(0, 2048, 20).astype(np.int32)
    m = hip_model(c1_model, max_seq=32, max_ctx=128)
    c = m.new_cache()
    o = OracleModel(c1_model)
    oc = o.new_cache(128)
    sampler = OracleSampler(2048, temperature=0.0, repeat_penalty=penalty, repeat_last_n=last_n)
    history = list(prompt)
    m.forward_prefill(c, prompt, logits=False)
    # Every prompt row gets an id on the device; the last row's is the first generated token.
    ol = o.forward(prompt, oc)[-1]
    hist_h = list(prompt)
    ids_h = m.greedy(len(prompt), [hist_h] * len(prompt), penalty, last_n)
    th = int(ids_h[-1])
    for step in range(64):
        to = sampler.sample(ol, np.array(history, np.int32))
        assert th == to, (step, th, to)
        history.append(to)
        hist_h.append(th)
        m.forward_prefill(c, [th], logits=False)
        th = int(m.greedy(1, [hist_h], penalty, last_n)[0])
        ol = o.forward([to], oc)[0]


def test_model_greedy_batch_rows_and_errors(H, c1_model):
    m = hip_model(c1_model, max_seq=32, max_ctx=64, max_batch=4, max_caches=4)
    with pytest.raises(H.HipError, match="no logits"):
        m.greedy(1)
    caches = [m.new_cache() for _ in range(3)]
    toks = np.array([5, 900, 2047], np.int32)
    for c, t in zip(caches, toks):
        m.forward_prefill(c, [t], logits=False)
    logits = m.forward_batch(caches, [1, 2, 3])
    ids = m.greedy(3)
    assert ids.tolist() == [greedy(row) for row in logits]
    with pytest.raises(H.HipError, match="no logits"):   # consumed
        m.greedy(3)
    m.forward_batch(caches, [4, 5, 6], logits=False)
    with pytest.raises(H.HipError, match="3 rows"):
        m.greedy(2)
    m.forward_batch(caches, [4, 5, 6], logits=False)
    with pytest.raises(H.HipError, match="exceeds"):
        m.greedy(3, [list(range(5000))] * 3, 1.1, 5000)


def test_model_greedy_after_every_pass_kind(H, c1_model):
    """forward, forward_prefill and forward_batch with the logits left in HBM: greedy gives
    the ids the host logits of the same pass give."""
    toks = np.array([3, 99, 1500, 7, 2047, 0], np.int32)
    a = hip_model(c1_model, max_seq=32, max_ctx=64, max_batch=4, max_caches=4)
    b = hip_model(c1_model, max_seq=32, max_ctx=64, max_batch=4, max_caches=4)
    want = [greedy(r) for r in a.forward(toks)]
    b.forward(toks, logits=False)
    assert b.greedy(len(toks)).tolist() == want
    ca, cb = a.new_cache(), b.new_cache()
    want = [greedy(r) for r in a.forward_prefill(ca, toks)]
    b.forward_prefill(cb, toks, logits=False)
    assert b.greedy(len(toks)).tolist() == want
    assert a.cache_pos(ca) == b.cache_pos(cb) == len(toks)
