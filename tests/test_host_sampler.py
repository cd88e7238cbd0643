"""The host stages of the device sampler (csrc/host/sampler.cpp, axon_sample_candidates and
axon_rng_*) against the oracle's sampler, which tests/test_oracle_sampling.py pins to the
reference's Sampler (src/sampling/sampler.cpp, rng.h) draw for draw and to the reference's own
sampler test cases. No GPU: the candidates come from a NumPy sort of the row, in the order the
device's top-k returns them (descending logits, equal logits by ascending id), on tie-free rows
where the reference's order is fixed too.

Bars: the generator's words and uniforms bit for bit; the drawn id and the generator state after
every draw identical to the oracle's."""
import numpy as np
import pytest

from test_oracle_sampling import OracleSampler


@pytest.fixture(scope="module")
def H():
    import axon_hip
    return axon_hip


@pytest.mark.parametrize("seed", [0, 1, 42, 2**63 + 5, 2**64 - 1])
def test_rng_matches_the_oracle(H, seed):
    a = H.Rng(seed)
    o = OracleSampler(4, seed=seed)
    from helpers import oracle
    import ctypes as C
    for _ in range(500):
        assert a.next() == oracle().ora_rng_next(C.byref(o.rng))
    for _ in range(500):
        assert a.uniform() == oracle().ora_rng_uniform(C.byref(o.rng))
    assert a.state() == tuple(o.rng.s)


CONFIGS = [
    dict(temperature=0.8, top_k=40, top_p=0.95, min_p=0.05),   # SamplerConfig's defaults
    dict(temperature=0.8, top_k=40, top_p=0.9, min_p=0.05),
    dict(temperature=1.5, top_k=256, top_p=1.0, min_p=0.0),    # the widest device top-k, no cuts
    dict(temperature=0.3, top_k=7, top_p=0.5, min_p=0.2),
    dict(temperature=1.0, top_k=1, top_p=0.95, min_p=0.05),    # one candidate
    dict(temperature=2.0, top_k=100, top_p=0.999, min_p=0.0),
]


def tie_free_row(rng, n, scale):
    return (rng.permutation(n).astype(np.float32) * np.float32(scale / n) - np.float32(scale / 2)) + \
        rng.standard_normal(n).astype(np.float32) * np.float32(1e-4)


@pytest.mark.parametrize("cfg", CONFIGS)
def test_host_stages_draw_as_the_oracle(H, cfg):
    n = 1000
    rng = np.random.default_rng(sum(int(v * 10) for v in cfg.values()))
    c = H.SamplerConfig(repeat_penalty=1.0, **cfg)
    mine = H.Rng(123)
    o = OracleSampler(n, repeat_penalty=1.0, seed=123, **cfg)
    kept = cfg["top_k"] if 0 < cfg["top_k"] < n else n
    for step in range(150):
        x = tie_free_row(rng, n, scale=[4.0, 12.0, 40.0][step % 3])
        assert len(np.unique(x)) == n
        order = np.lexsort((np.arange(n), -x))[:kept]
        got = H.sample_candidates(c, mine, x[order], order)
        want = o.sample(x)
        assert got == want, (step, got, want)
        assert mine.state() == tuple(o.rng.s)


def test_host_stages_reject_greedy_and_empty(H):
    with pytest.raises(H.HipError, match="temperature"):
        H.sample_candidates(H.SamplerConfig(temperature=0.0), H.Rng(1), [1.0], [0])
    with pytest.raises(H.HipError, match="n >= 1"):
        H.sample_candidates(H.SamplerConfig(), H.Rng(1), np.zeros(0, np.float32), np.zeros(0, np.int32))
