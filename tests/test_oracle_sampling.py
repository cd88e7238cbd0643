"""The oracle's sampler (oracle/model.c: ora_repeat_penalty, ora_sample, ora_rng_*), restated from
src/sampling/sampler.cpp and src/sampling/rng.h, pinned three ways:

* the reference's own sampler test cases (tests/unit/test_sampler.cpp:35-135) as known answers;
* what the mathematics fixes: greedy is numpy's first-maximum argmax on NaN-free rows, hand-worked
  NaN rows follow max_element's `<` scan, and a one-id window rescales exactly one logit;
* the reference's own Sampler compiled under oracle/_ref, draw for draw with the same seed.

The device greedy step (tests/test_hip_sampling.py) is checked against this oracle."""
import ctypes as C

import numpy as np
import pytest

from helpers import have_ref, oracle, ref

NAN = float("nan")


class Config(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_k", C.c_int), ("top_p", C.c_float), ("min_p", C.c_float),
                ("repeat_penalty", C.c_float), ("repeat_last_n", C.c_int)]


class Rng(C.Structure):
    _fields_ = [("s", C.c_uint64 * 4)]


class OracleSampler:
    """ora_sample with its scratch, as Sampler holds it (sampler.cpp:17-26)."""

    def __init__(self, n_vocab, temperature=0.8, top_k=40, top_p=0.95, min_p=0.05, repeat_penalty=1.1,
                 repeat_last_n=64, seed=1):
        self.n = n_vocab
        self.cfg = Config(temperature, top_k, top_p, min_p, repeat_penalty, repeat_last_n)
        self.rng = Rng()
        oracle().ora_rng_seed(C.byref(self.rng), C.c_uint64(seed))
        self.sl = np.zeros(n_vocab, np.float32)
        self.order = np.zeros(n_vocab, np.int32)
        self.probs = np.zeros(n_vocab, np.float64)
        self.touched = np.zeros(n_vocab, np.uint8)

    def sample(self, logits, recent=()):
        x = np.ascontiguousarray(logits, np.float32)
        r = np.ascontiguousarray(recent, np.int32)
        return oracle().ora_sample(C.byref(self.cfg), C.byref(self.rng), x.ctypes.data_as(C.c_void_p),
                                   C.c_int32(self.n), r.ctypes.data_as(C.c_void_p), C.c_size_t(len(r)),
                                   self.sl.ctypes.data_as(C.c_void_p), self.order.ctypes.data_as(C.c_void_p),
                                   self.probs.ctypes.data_as(C.c_void_p), self.touched.ctypes.data_as(C.c_void_p))


def greedy(logits, recent=(), penalty=1.0, last_n=64):
    return OracleSampler(len(logits), temperature=0.0, repeat_penalty=penalty, repeat_last_n=last_n).sample(
        logits, recent)


def penalize(logits, recent, penalty, last_n):
    x = np.array(logits, np.float32)
    r = np.ascontiguousarray(recent, np.int32)
    touched = np.zeros(len(x), np.uint8)
    oracle().ora_repeat_penalty(x.ctypes.data_as(C.c_void_p), C.c_size_t(len(x)), r.ctypes.data_as(C.c_void_p),
                                C.c_size_t(len(r)), C.c_float(penalty), C.c_int(last_n),
                                touched.ctypes.data_as(C.c_void_p))
    assert not touched.any()
    return x


# ---- known answers: tests/unit/test_sampler.cpp ---------------------------------------------


def test_rng_known_properties():
    # test_sampler.cpp:35-58: deterministic per seed, different across seeds, uniforms in [0, 1).
    a, b, c = Rng(), Rng(), Rng()
    oracle().ora_rng_seed(C.byref(a), C.c_uint64(42))
    oracle().ora_rng_seed(C.byref(b), C.c_uint64(42))
    oracle().ora_rng_seed(C.byref(c), C.c_uint64(43))
    xs = [oracle().ora_rng_next(C.byref(a)) for _ in range(100)]
    assert xs == [oracle().ora_rng_next(C.byref(b)) for _ in range(100)]
    assert xs != [oracle().ora_rng_next(C.byref(c)) for _ in range(100)]
    us = [oracle().ora_rng_uniform(C.byref(a)) for _ in range(1000)]
    assert all(0.0 <= u < 1.0 for u in us)


def test_temperature_zero_is_greedy():
    # test_sampler.cpp:60-66.
    s = OracleSampler(8, temperature=0.0, top_k=1, top_p=0.1, seed=7)
    logits = [0.1, 2.0, 0.5, 9.0, -1.0, 3.0, 0.0, 8.9]
    assert all(s.sample(logits) == 3 for _ in range(10))


def test_repetition_penalty_known_answers():
    # test_sampler.cpp:114-135.
    logits = [1.0, 1.2, 0.0, 0.0, 0.0, 0.0, 0.0, 0.0]
    assert greedy(logits, [], 1.5, 4) == 1
    assert greedy(logits, [1, 1, 1], 1.5, 4) == 0            # 1.2 / 1.5 = 0.8 < 1.0
    assert greedy(logits, [1, 5, 6, 7, 2], 1.5, 4) == 1      # 1 is outside the window of 4
    negatives = [-1.0, -0.5, -3.0, -3.0, -3.0, -3.0, -3.0, -3.0]
    assert greedy(negatives, [1], 2.5, 4) == 0               # -0.5 * 2.5 = -1.25 < -1.0
    assert greedy(logits, [1, 1, 1, 1], 1.05, 4) == 1        # once per distinct token


def test_top_k_top_p_min_p_support():
    # test_sampler.cpp:68-112: the set of tokens each stage can still produce.
    def support(s, logits, draws=2000):
        return {s.sample(logits) for _ in range(draws)}

    logits = [0.0, 1.0, 2.0, 3.0, 4.0, 5.0, 6.0, 7.0]
    s = OracleSampler(8, temperature=1.0, top_k=3, top_p=1.0, min_p=0.0, repeat_penalty=1.0, seed=1)
    assert support(s, logits) == {5, 6, 7}
    logits = [3.0, 2.0, 1.0, -20.0, -20.0, -20.0, -20.0, -20.0]
    narrow = OracleSampler(8, temperature=1.0, top_k=0, top_p=0.6, min_p=0.0, repeat_penalty=1.0, seed=1)
    assert support(narrow, logits) == {0}
    wider = OracleSampler(8, temperature=1.0, top_k=0, top_p=0.8, min_p=0.0, repeat_penalty=1.0, seed=1)
    assert support(wider, logits) == {0, 1}
    mp = OracleSampler(8, temperature=1.0, top_k=0, top_p=1.0, min_p=0.2, repeat_penalty=1.0, seed=1)
    assert support(mp, logits) == {0, 1}


# ---- what the mathematics fixes ---------------------------------------------------------------


def test_greedy_is_first_maximum_on_nan_free_rows():
    rng = np.random.default_rng(0)
    for trial in range(200):
        n = int(rng.integers(1, 300))
        # Small integers give many ties; the first maximum must win.
        x = rng.integers(-4, 5, n).astype(np.float32) if trial % 2 else rng.standard_normal(n).astype(np.float32)
        assert greedy(x) == int(np.argmax(x))


@pytest.mark.parametrize("row, want", [
    ([NAN, 1.0, 2.0], 0),                 # a NaN first element is never replaced
    ([1.0, NAN, 2.0], 2),                 # a later NaN is skipped
    ([1.0, 3.0, NAN, 3.0], 1),
    ([NAN, NAN, NAN], 0),
    ([-0.0, 0.0], 0),                     # -0 == +0: the first wins
    ([0.0, -0.0, 0.0], 0),
    ([-np.inf, -np.inf], 0),
    ([1.0, np.inf, np.inf], 1),
    ([-np.inf, NAN, -3.0], 2),
])
def test_greedy_nan_and_signed_zero_rows(row, want):
    assert greedy(row) == want


def test_penalty_rescales_each_distinct_id_once():
    x = np.array([2.0, -2.0, 3.0, 0.0, 5.0], np.float32)
    got = penalize(x, [0, 1, 0, 1, 3, 9, -1], 4.0, 64)
    assert got.tolist() == [0.5, -8.0, 3.0, 0.0, 5.0]
    # The window is the last repeat_last_n ids; repeat_last_n 0 or penalty 1 turn it off.
    assert penalize(x, [0, 2], 4.0, 1).tolist() == [2.0, -2.0, 0.75, 0.0, 5.0]
    assert np.array_equal(penalize(x, [0, 2], 4.0, 0), x)
    assert np.array_equal(penalize(x, [0, 2], 1.0, 64), x)


# ---- the reference's own Sampler ----------------------------------------------------------------


def ref_sample(logits, recent, temperature, top_k, top_p, min_p, penalty, last_n, seed, draws):
    x = np.ascontiguousarray(logits, np.float32)
    r = np.ascontiguousarray(recent, np.int32)
    out = np.zeros(draws, np.int32)
    ref().ref_sample(x.ctypes.data_as(C.c_void_p), C.c_size_t(len(x)), r.ctypes.data_as(C.c_void_p),
                     C.c_size_t(len(r)), C.c_float(temperature), C.c_int(top_k), C.c_float(top_p),
                     C.c_float(min_p), C.c_float(penalty), C.c_int(last_n), C.c_uint64(seed), C.c_size_t(draws),
                     out.ctypes.data_as(C.c_void_p))
    return out.tolist()


needs_ref = pytest.mark.skipif(not have_ref(), reason="oracle/_ref not built (no reference checkout)")


@needs_ref
@pytest.mark.parametrize("case", range(24))
def test_sampler_matches_reference_draw_for_draw(case):
    rng = np.random.default_rng(100 + case)
    n = int(rng.choice([8, 100, 2048, 32000]))
    # Distinct logits: the reference's partial_sort leaves equal logits in an unspecified order.
    x = rng.permutation(n).astype(np.float32) * np.float32(rng.uniform(0.001, 0.05))
    x = (x - x.mean()).astype(np.float32)
    recent = rng.integers(-2, n + 2, int(rng.integers(0, 200))).astype(np.int32)
    temperature = float(rng.choice([0.0, 0.0, 0.5, 0.8, 1.3]))
    top_k = int(rng.choice([0, 1, 5, 40]))
    top_p = float(rng.choice([1.0, 0.9, 0.5]))
    min_p = float(rng.choice([0.0, 0.05, 0.2]))
    penalty = float(rng.choice([1.0, 1.1, 1.5, 0.8]))
    last_n = int(rng.choice([0, 4, 64, 512]))
    seed = int(rng.integers(1, 2**62))
    draws = 50
    o = OracleSampler(n, temperature, top_k, top_p, min_p, penalty, last_n, seed)
    want = ref_sample(x, recent, temperature, top_k, top_p, min_p, penalty, last_n, seed, draws)
    assert [o.sample(x, recent) for _ in range(draws)] == want


@needs_ref
def test_greedy_matches_reference_on_nan_and_tie_rows():
    rows = [[NAN, 1.0, 2.0], [1.0, NAN, 2.0], [NAN] * 4, [-0.0, 0.0], [2.0, 5.0, 5.0, 1.0], [3.0]]
    for row in rows:
        assert greedy(row) == ref_sample(row, [], 0.0, 40, 0.95, 0.05, 1.0, 64, 1, 1)[0], row
    rng = np.random.default_rng(9)
    for _ in range(50):
        x = rng.integers(-3, 4, 64).astype(np.float32)
        recent = rng.integers(0, 64, 20).astype(np.int32)
        assert greedy(x, recent, 1.3, 16) == ref_sample(x, recent, 0.0, 40, 0.95, 0.05, 1.3, 16, 1, 1)[0]
