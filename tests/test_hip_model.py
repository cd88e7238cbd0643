"""The device-resident forward pass (libaxon_host.so driving the hip table) against the CPU oracle's
forward pass, which is itself bit-identical to the reference's LlamaModel on the scalar table
(tests/test_oracle_ref.py). Patterned on the reference's model tests:
test_model_forward.cpp:40-54 (logits of the synthetic F32 model against the NumPy fixture),
test_model_kernels.cpp:59-90 (a second table against the scalar table on the quantized files),
test_model_cached.cpp:60-106 (cached decoding equals the full pass), test_model_batch.cpp:103-157
(batched rows equal each sequence alone) and test_model_batch.cpp:209-253 (forward_batch bounds).

The north star's bars: logits within 1e-4 max-abs of the scalar table, greedy tokens identical
over 64 steps. Matmuls and quantization are bit-exact here, so logits match the oracle's bits
except where an exp or cos rounds differently in its last bit."""
from dataclasses import replace

import numpy as np
import pytest

from helpers import GOLDEN, OracleModel, golden

pytestmark = pytest.mark.gpu

FIXTURES = ["synthetic-2l.gguf", "synthetic-2l-q8_0.gguf", "synthetic-2l-q4_0.gguf", "synthetic-2l-q4_1.gguf"]


def hip_model(path, **kw):
    import axon_hip as H
    return H.Model(path, **kw)


@pytest.fixture(scope="module")
def tokens():
    return golden("model/synthetic-2l.tokens.axt").ravel().astype(np.int32)


@pytest.mark.parametrize("name", FIXTURES)
def test_forward_matches_oracle(name, tokens):
    path = GOLDEN / "gguf" / name
    m = hip_model(path, max_seq=32, max_ctx=64)
    assert m.table_name == "hip"
    got = m.forward(tokens)
    want = OracleModel(path).forward(tokens)
    assert np.max(np.abs(got - want)) <= 1e-4
    assert np.mean(got == want) > 0.99, np.mean(got == want)


def test_f32_model_matches_numpy_fixture(tokens):
    m = hip_model(GOLDEN / "gguf" / "synthetic-2l.gguf", max_seq=32, max_ctx=64)
    want = golden("model/synthetic-2l.logits.axt")
    assert np.max(np.abs(m.forward(tokens) - want.reshape(len(tokens), -1))) < 1e-4


@pytest.mark.parametrize("name", FIXTURES)
def test_cached_decoding_equals_full_pass(name, tokens):
    m = hip_model(GOLDEN / "gguf" / name, max_seq=32, max_ctx=64)
    full = m.forward(tokens)
    c = m.new_cache()
    out = [m.forward_prefill(c, tokens[:8])]
    for t in tokens[8:]:
        out.append(m.forward_prefill(c, [t]))
    assert m.cache_pos(c) == len(tokens)
    assert np.array_equal(np.concatenate(out), full)


@pytest.mark.parametrize("name", ["synthetic-2l-q4_0.gguf", "synthetic-2l.gguf"])
def test_batched_rows_equal_each_sequence_alone(name, tokens):
    path = GOLDEN / "gguf" / name
    m = hip_model(path, max_seq=32, max_ctx=64, max_batch=4, max_caches=8)
    lens = [3, 7, 11]
    alone = []
    caches = []
    for i, n in enumerate(lens):
        c = m.new_cache()
        m.forward_prefill(c, tokens[i:i + n])
        caches.append(c)
    nxt = np.array([tokens[20], tokens[21], tokens[22]], np.int32)
    batch = m.forward_batch(caches, nxt)
    for i, n in enumerate(lens):
        c = m.new_cache()
        m.forward_prefill(c, tokens[i:i + n])
        alone.append(m.forward_prefill(c, [nxt[i]])[0])
    assert np.array_equal(batch, np.stack(alone))
    assert [m.cache_pos(c) for c in caches] == [n + 1 for n in lens]


def test_forward_batch_bounds(tokens):
    import axon_hip as H
    m = hip_model(GOLDEN / "gguf" / "synthetic-2l-q4_0.gguf", max_seq=8, max_ctx=16, max_batch=2, max_caches=4)
    a, b, c = m.new_cache(), m.new_cache(), m.new_cache()
    with pytest.raises(H.HipError, match="exceed max_batch"):
        m.forward_batch([a, b, c], [1, 2, 3])
    with pytest.raises(H.HipError, match="appears twice"):
        m.forward_batch([a, a], [1, 2])
    with pytest.raises(H.HipError, match="outside the vocabulary"):
        m.forward_batch([a, b], [1, 100000])
    with pytest.raises(H.HipError, match="exceed max_seq"):
        m.forward_prefill(a, np.arange(9))
    m.forward_prefill(a, np.arange(8))
    m.forward_prefill(a, np.arange(8))
    with pytest.raises(H.HipError, match="context overflow"):
        m.forward_batch([a, b], [1, 2])
    with pytest.raises(H.HipError, match="context overflow"):
        m.forward_prefill(a, [1])


def test_kv_cache_rows_match_oracle_cache(tokens):
    # The cache write (bias, RoPE, copy at the row's position) reproduces the oracle's K and V.
    path = GOLDEN / "gguf" / "synthetic-2l-q8_0.gguf"
    m = hip_model(path, max_seq=32, max_ctx=64)
    c = m.new_cache()
    m.forward_prefill(c, tokens[:10])
    o = OracleModel(path)
    oc = o.new_cache(64)
    o.forward(tokens[:10], oc)
    row = o.cfg.n_head_kv * o.cfg.head_dim
    store = oc._store.reshape(o.cfg.n_layer, 2, 64, row)
    for layer in range(o.cfg.n_layer):
        assert np.array_equal(m.cache_rows(c, layer, False, 10), store[layer, 0, :10])
        assert np.array_equal(m.cache_rows(c, layer, True, 10), store[layer, 1, :10])


def _greedy(step, first_logits, n):
    out = []
    logits = first_logits
    for _ in range(n):
        t = int(np.argmax(logits))
        out.append(t)
        logits = step(t)
    return out


@pytest.mark.parametrize("cfg", ["c1", "c4", "c5"])
def test_greedy_64_tokens_identical_on_config_shapes(cfg, tmp_path_factory):
    """The BASELINE shapes at full width with 2 layers and a 2048-token vocabulary: 64 greedy
    decode steps after a 24-token prompt give the same tokens as the oracle, every logit within
    1e-4."""
    import synth
    spec = replace(synth.CONFIGS[cfg], name=f"t-{cfg}-2l", n_layer=2, n_vocab=2048, seed=11)
    path = synth.cached_model(spec, tmp_path_factory.mktemp("models"))
    prompt = np.random.default_rng(5).integers(0, spec.n_vocab, 24).astype(np.int32)
    m = hip_model(path, max_seq=32, max_ctx=128)
    c = m.new_cache()
    o = OracleModel(path)
    oc = o.new_cache(128)
    hl = m.forward_prefill(c, prompt)
    ol = o.forward(prompt, oc)
    assert np.max(np.abs(hl - ol)) <= 1e-4
    diffs = []

    def hstep(t):
        return m.forward_prefill(c, [t])[0]

    def ostep(t):
        logits = o.forward([t], oc)[0]
        return logits

    h_tokens, o_tokens = [], []
    hlog, olog = hl[-1], ol[-1]
    for _ in range(64):
        th, to = int(np.argmax(hlog)), int(np.argmax(olog))
        h_tokens.append(th)
        o_tokens.append(to)
        assert th == to, (len(h_tokens), h_tokens[-5:], o_tokens[-5:])
        hlog, olog = hstep(th), ostep(to)
        diffs.append(float(np.max(np.abs(hlog - olog))))
    assert max(diffs) <= 1e-4, max(diffs)
