"""The device sampler (sampling.hip: axon_hip_repeat_penalty_rows, axon_hip_argmax_rows,
axon_hip_topk_rows, axon_hip_sort_rows, and the model's axon_model_greedy and axon_model_sample) against the oracle's
sampler, which tests/test_oracle_sampling.py pins to the reference's Sampler draw for draw.

Selection is index work, so the bar is bit-exact: the same id for every row, the penalised
logits bit-identical to the oracle's, and for the stochastic stages the same draws and generator
states. Greedy rows cover the full Llama-3 vocabulary (128256), widths around the kernel's 64-way
split (1, 63, 64, 65, 4097), ties placed across split boundaries, NaN (first element and
elsewhere), signed zeros, infinities and strided rows. Top-k rows cover the Qwen2.5 and Llama-3
vocabularies, k of 1, 40 and 256, ties, NaN, signed zeros, and rows laid out so that one thread's
stride holds the largest values (the kernel's later rounds)."""
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


# ---- top-k candidates and the stochastic sampler ----------------------------------------------

def topk_reference(x, k):
    """The kernel's contract: the k largest non-NaN values, descending, equal values by
    ascending index (-0 equal to +0), ids -1 past the non-NaN values."""
    n = len(x)
    ok = ~np.isnan(x)
    idx = np.nonzero(ok)[0]
    v = x[idx] + np.float32(0.0)  # -0 -> +0
    order = idx[np.lexsort((idx, -v))][:k]
    ids = np.full(k, -1, np.int32)
    ids[:len(order)] = order
    vals = np.zeros(k, np.float32)
    vals[:len(order)] = x[order]
    return vals, ids


def topk_rows(kind, n, rng):
    x = rng.standard_normal(n).astype(np.float32) * np.float32(3.0)
    if kind == "ties":
        x = np.round(x * 2) / 2          # a handful of distinct values
    elif kind == "nan":
        x[rng.integers(0, n, n // 5)] = NAN
    elif kind == "zeros":
        x = -np.abs(x) - 1
        x[rng.integers(0, n, 30)] = np.float32(-0.0)
        x[rng.integers(0, n, 30)] = np.float32(0.0)
    elif kind == "equal":
        x[:] = np.float32(0.25)
    elif kind == "one-stride":          # every large value in one thread's stride of 1024
        x[5::1024] = np.float32(100.0) + np.arange(len(x[5::1024]), dtype=np.float32)
    elif kind == "ascending":
        x = np.sort(x)
    elif kind == "descending":
        x = np.sort(x)[::-1].copy()
    return x.astype(np.float32)


@pytest.mark.parametrize("n", [151936, 128256, 4097, 300, 40])
@pytest.mark.parametrize("k", [1, 40, 256])
def test_topk_rows_match_sorted_order(H, n, k):
    if k > n:
        pytest.skip("k above the row length is refused")
    kinds = ["normal", "ties", "nan", "zeros", "equal", "one-stride", "ascending", "descending"]
    rng = np.random.default_rng(n + k)
    x = np.stack([topk_rows(kind, n, rng) for kind in kinds])
    stride = n + 3
    xs = np.zeros((len(kinds), stride), np.float32)
    xs[:, :n] = x
    dx = H.DeviceBuffer.of(xs)
    ol = H.DeviceBuffer(4 * len(kinds) * k)
    oi = H.DeviceBuffer(4 * len(kinds) * k)
    H.call("topk_rows", dx, n, len(kinds), stride, k, ol, oi)
    got_v = ol.download(np.float32, len(kinds) * k).reshape(len(kinds), k)
    got_i = oi.download(np.int32, len(kinds) * k).reshape(len(kinds), k)
    for r, kind in enumerate(kinds):
        want_v, want_i = topk_reference(x[r], k)
        assert np.array_equal(got_i[r], want_i), (kind, np.nonzero(got_i[r] != want_i)[0][:5])
        assert np.array_equal(got_v[r].view(np.uint32), want_v.view(np.uint32)), kind


def test_topk_rows_bounds(H):
    dx = H.DeviceBuffer.of(np.zeros(300, np.float32))
    out = H.DeviceBuffer(4 * 300)
    with pytest.raises(H.HipError, match="k"):
        H.call("topk_rows", dx, 300, 1, 300, 257, out, out)
    with pytest.raises(H.HipError, match="k"):
        H.call("topk_rows", dx, 30, 1, 30, 31, out, out)
    with pytest.raises(H.HipError, match="stride"):
        H.call("topk_rows", dx, 300, 1, 200, 4, out, out)


ROW_CONFIGS = [
    dict(temperature=0.8, top_k=40, top_p=0.95, min_p=0.05, repeat_penalty=1.1, repeat_last_n=64),
    dict(temperature=0.8, top_k=40, top_p=0.9, min_p=0.05, repeat_penalty=1.0, repeat_last_n=64),
    dict(temperature=0.0, top_k=40, top_p=0.95, min_p=0.05, repeat_penalty=1.3, repeat_last_n=16),
    dict(temperature=1.0, top_k=1, top_p=0.95, min_p=0.05, repeat_penalty=1.1, repeat_last_n=64),
    dict(temperature=1.7, top_k=256, top_p=1.0, min_p=0.0, repeat_penalty=1.5, repeat_last_n=8),
]


def test_model_sample_matches_oracle_sampler(H, c1_model):
    """Five sequences decoded together for 24 steps, each row with its own sampler settings and
    generator (greedy with a penalty among them): every drawn id and every generator state
    equal the oracle sampler's on the host logits of the same pass."""
    n_seq = len(ROW_CONFIGS)
    m = hip_model(c1_model, max_seq=32, max_ctx=128, max_batch=n_seq, max_caches=n_seq)
    rng = np.random.default_rng(21)
    prompts = [rng.integers(0, 2048, 6 + 3 * i).astype(np.int32) for i in range(n_seq)]
    caches = [m.new_cache() for _ in range(n_seq)]
    hist = [list(p) for p in prompts]
    cfgs = [H.SamplerConfig(**c) for c in ROW_CONFIGS]
    gens = [H.Rng(1000 + i) for i in range(n_seq)]
    orc = [OracleSampler(2048, seed=1000 + i, **c) for i, c in enumerate(ROW_CONFIGS)]
    for i in range(n_seq):
        m.forward_prefill(caches[i], prompts[i][:-1], logits=False)
    toks = [int(p[-1]) for p in prompts]
    for step in range(24):
        logits = m.forward_batch(caches, toks)
        got = m.sample(cfgs, gens, hist)
        want = [orc[i].sample(logits[i], np.array(hist[i], np.int32)) for i in range(n_seq)]
        assert got.tolist() == want, (step, got.tolist(), want)
        for i in range(n_seq):
            assert gens[i].state() == tuple(orc[i].rng.s), (step, i)
            hist[i].append(int(got[i]))
        toks = [int(t) for t in got]


def test_model_sample_bounds(H, c1_model):
    m = hip_model(c1_model, max_seq=32, max_ctx=64, max_batch=2, max_caches=2)
    c = m.new_cache()
    with pytest.raises(H.HipError, match="no logits"):
        m.sample([H.SamplerConfig()], [H.Rng(1)])
    m.forward_prefill(c, [1, 2, 3], logits=False)
    with pytest.raises(H.HipError, match="3 rows"):
        m.sample([H.SamplerConfig()], [H.Rng(1)])
    g = H.Rng(5)
    before = g.state()
    with pytest.raises(H.HipError, match="3 rows"):
        m.sample([H.SamplerConfig(top_k=0)] * 2, [g, H.Rng(6)])
    assert g.state() == before  # nothing ran
    # The pass's logits are still there after a refused call.
    ids = m.sample([H.SamplerConfig(temperature=0.0)] * 3, [H.Rng(1)] * 3)
    assert len(ids) == 3


@pytest.mark.parametrize("n", [151936, 128256, 32000, 4097, 1025, 1024, 300, 40, 1])
def test_sort_rows_match_sorted_order(H, n):
    """The whole-row sort behind top_k 0: every row kind of the top-k test, every position in the
    order the top-k kernel keeps (NaN last with ids -1 and logits 0), values bit for bit (signed
    zeros kept), at row lengths around one 1024-key group and at the largest vocabularies."""
    kinds = ["normal", "ties", "nan", "zeros", "equal", "one-stride", "ascending", "descending"]
    rng = np.random.default_rng(n)
    x = np.stack([topk_rows(kind, n, rng) for kind in kinds])
    stride = n + 5
    xs = np.zeros((len(kinds), stride), np.float32)
    xs[:, :n] = x
    H.lib().axon_hip_sort_rows_work_bytes.restype = C.c_size_t
    work = H.DeviceBuffer(H.lib().axon_hip_sort_rows_work_bytes(C.c_size_t(n), C.c_size_t(len(kinds))))
    dx = H.DeviceBuffer.of(xs)
    ol = H.DeviceBuffer(4 * len(kinds) * n)
    oi = H.DeviceBuffer(4 * len(kinds) * n)
    H.call("sort_rows", dx, n, len(kinds), stride, work, ol, oi)
    got_v = ol.download(np.float32, len(kinds) * n).reshape(len(kinds), n)
    got_i = oi.download(np.int32, len(kinds) * n).reshape(len(kinds), n)
    for r, kind in enumerate(kinds):
        want_v, want_i = topk_reference(x[r], n)
        assert np.array_equal(got_i[r], want_i), (kind, np.nonzero(got_i[r] != want_i)[0][:5])
        assert np.array_equal(got_v[r].view(np.uint32), want_v.view(np.uint32)), kind


def test_sort_rows_bounds(H):
    dx = H.DeviceBuffer.of(np.zeros(300, np.float32))
    out = H.DeviceBuffer(4 * 300)
    with pytest.raises(H.HipError, match="stride"):
        H.call("sort_rows", dx, 300, 1, 200, out, out, out)
    with pytest.raises(H.HipError, match="stride"):
        H.call("sort_rows", dx, 0, 1, 300, out, out, out)
    with pytest.raises(H.HipError, match="required"):
        H.call("sort_rows", dx, 300, 1, 300, None, out, out)


WHOLE_CONFIGS = [
    dict(temperature=0.8, top_k=0, top_p=0.95, min_p=0.05, repeat_penalty=1.1, repeat_last_n=64),
    dict(temperature=1.3, top_k=0, top_p=1.0, min_p=0.0, repeat_penalty=1.0, repeat_last_n=64),
    dict(temperature=0.9, top_k=300, top_p=0.98, min_p=0.0, repeat_penalty=1.2, repeat_last_n=32),
    dict(temperature=0.8, top_k=40, top_p=0.95, min_p=0.05, repeat_penalty=1.1, repeat_last_n=64),
    dict(temperature=0.0, top_k=0, top_p=0.95, min_p=0.05, repeat_penalty=1.3, repeat_last_n=16),
    dict(temperature=2.0, top_k=0, top_p=0.5, min_p=0.01, repeat_penalty=1.1, repeat_last_n=64),
]


def test_model_sample_whole_vocabulary_matches_oracle_sampler(H, c1_model):
    """top_k 0 (sampler.cpp:115-117 sorts every id) beside top_k 300 and 40 and a greedy row, six
    sequences for 24 steps, then the same with fewer rows (the device room of the first call
    serves): every drawn id and generator state equal the oracle sampler's, whose qsort of the
    whole vocabulary is the reference's sort."""
    n_seq = len(WHOLE_CONFIGS)
    m = hip_model(c1_model, max_seq=32, max_ctx=128, max_batch=n_seq, max_caches=n_seq)
    rng = np.random.default_rng(22)
    prompts = [rng.integers(0, 2048, 5 + 2 * i).astype(np.int32) for i in range(n_seq)]
    caches = [m.new_cache() for _ in range(n_seq)]
    hist = [list(p) for p in prompts]
    cfgs = [H.SamplerConfig(**c) for c in WHOLE_CONFIGS]
    gens = [H.Rng(2000 + i) for i in range(n_seq)]
    orc = [OracleSampler(2048, seed=2000 + i, **c) for i, c in enumerate(WHOLE_CONFIGS)]
    for i in range(n_seq):
        m.forward_prefill(caches[i], prompts[i][:-1], logits=False)
    toks = [int(p[-1]) for p in prompts]
    for step in range(24):
        rows = n_seq if step < 16 else 2  # the last steps decode two sequences only
        logits = m.forward_batch(caches[:rows], toks[:rows])
        got = m.sample(cfgs[:rows], gens[:rows], hist[:rows])
        want = [orc[i].sample(logits[i], np.array(hist[i], np.int32)) for i in range(rows)]
        assert got.tolist() == want, (step, got.tolist(), want)
        for i in range(rows):
            assert gens[i].state() == tuple(orc[i].rng.s), (step, i)
            hist[i].append(int(got[i]))
        toks[:rows] = [int(t) for t in got]
